/*
 * exl3_hip.h -- C ABI of the MI355X (gfx950) EXL3 quantized-linear library.
 *
 * Drop-in boundary for the reference engine's EXL3 operator API.  The
 * reference dispatches every EXL3 projection through
 *   Exl3Linear::new      native/src/linear.rs:577-653
 *   Exl3Linear::forward  native/src/linear.rs:731-998
 *   Exl3Group::forward   native/src/linear.rs:2382
 *   Exl3SwitchGlu        native/src/moe.rs:611-1085 (forward :905-975)
 * which reach the GPU through the generic C entry point
 *   int mlxl3_metal_kernel(...)   native/ffi/mlx_bridge.cpp:860-911
 * with errors as int status + a thread-local message (mlxl3_mlx_error,
 * mlx_bridge.cpp:49-66, :176).  This header replaces that boundary with typed
 * entry points; the calling conventions are kept: int status, thread-local
 * error text, dtype codes of mlx_bridge.cpp:71-80, codebook codes of
 * native/src/codec.rs:5-23.
 *
 * Memory: every pointer is a device pointer owned by the caller (hipMalloc or
 * any allocator of device memory).  Handles borrow the weight buffers and hold
 * only shapes and launch parameters, so the buffers must outlive the handle.
 * Execution is asynchronous on the given stream (a hipStream_t passed as
 * void*, NULL for the default stream); the caller synchronises.
 *
 * Workspace: forward calls take a caller-owned device workspace of at least
 * *_workspace_bytes(rows) bytes.  A workspace must be zero-filled once before
 * its first use (exl3_workspace_init does that on a stream); every call leaves
 * it reusable by any entry point (its first 64 KiB hold counters that every
 * call leaves at zero).  Calls that share one workspace must not run
 * concurrently.
 *
 * Threading: handles are immutable after creation and may be used from any
 * thread; error messages are per thread.
 */
#ifndef EXL3_HIP_H
#define EXL3_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  EXL3_OK = 0,
  EXL3_EINVAL = -1,      /* bad argument or shape (nothing launched) */
  EXL3_EDEVICE = -2,     /* HIP runtime / launch error */
  EXL3_ENOMEM = -3,      /* host allocation failed */
  EXL3_EUNSUPPORTED = -4 /* valid request outside this build */
} exl3_status;

/* dtype codes of mlx_bridge.cpp:71-80 */
typedef enum { EXL3_F16 = 9, EXL3_F32 = 10, EXL3_BF16 = 12 } exl3_dtype;

/* codec.rs:5-23: Default (3INST), Mcg, Mul1 */
typedef enum { EXL3_CB_3INST = 0, EXL3_CB_MCG = 1, EXL3_CB_MUL1 = 2 } exl3_codebook;

typedef struct exl3_linear exl3_linear;
typedef struct exl3_moe exl3_moe;

/* Message of the last failed call on this thread ("" if none).
 * Replaces mlxl3_mlx_error, mlx_bridge.cpp:176. */
const char* exl3_last_error(void);

/* Library version string. */
const char* exl3_version(void);

/* Exl3Linear::new, linear.rs:577-653.  trellis: [in/16][out/16][16k] u16
 * (I16 accepted by the caller's reinterpretation); suh f16[in]; svh f16[out];
 * bias f16[out] or NULL; k in 1..8; cb an exl3_codebook.  in and out must be
 * positive multiples of 128 (linear.rs:593-596).  A trellis of 4 GiB or more
 * (in * out * k / 8 bytes) is rejected: the kernels address it with 32-bit
 * offsets (no counterpart in the reference, whose largest real tensors are
 * ~1.2 GB). */
int exl3_linear_create(const uint16_t* trellis, int32_t in, int32_t out, int32_t k, int32_t cb,
                       const uint16_t* suh, const uint16_t* svh, const uint16_t* bias,
                       exl3_linear** out_handle);
void exl3_linear_destroy(exl3_linear* handle);

/* Input / output features of a handle (Exl3Linear::input_dims/output_dims,
 * linear.rs:655-660). */
int32_t exl3_linear_in_features(const exl3_linear* handle);
int32_t exl3_linear_out_features(const exl3_linear* handle);

/* Workspace needed by exl3_linear_forward for `rows` activation rows. */
size_t exl3_linear_workspace_bytes(const exl3_linear* handle, int64_t rows);

/* Zero-fills a workspace with a kernel on `stream` (no hipMemset, so it may
 * be recorded into a graph). */
int exl3_workspace_init(void* workspace, size_t bytes, void* stream);

/* Output dtype of a projection for activations of x_type (linear.rs:992-995:
 * y.astype(x.dtype) + bias with the f16 bias under MLX's type promotion):
 * x_type without a bias; with a bias f16 -> f16, f32 -> f32 and bf16 -> f32
 * (MLX promotes bfloat16 + float16 to float32).  -1 for a null handle or an
 * unknown dtype. */
int32_t exl3_linear_output_dtype(const exl3_linear* handle, int32_t x_type);

/* Exl3Linear::forward, linear.rs:731-998: y[rows][out] = EXL3 linear of
 * x[rows][in].  x_type: exl3_dtype; y_type must equal
 * exl3_linear_output_dtype(handle, x_type) (EXL3_EINVAL otherwise): the f16
 * result is cast to x's dtype, then the bias is added in the promoted dtype.
 * rows >= 1.  rows <= 16 runs the fused multi-row QMV (one launch); larger
 * rows run the prologue and the QMM. */
int exl3_linear_forward(const exl3_linear* handle, const void* x, int32_t x_type, int64_t rows,
                        void* y, int32_t y_type, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Allocation-free exl3_linear_forward (no counterpart in the reference: for
 * callers that cannot allocate -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The same kernels and results as
 * exl3_linear_forward, with its workspace taken from a fixed device array of
 * exl3_linear_noalloc_max_bytes() bytes that the library holds on every GPU
 * it runs on until the process ends; no hipMalloc, hipFree or allocating
 * library routine is called.  Calls whose workspace
 * (exl3_linear_workspace_bytes) exceeds that size fail with
 * EXL3_EUNSUPPORTED before any launch.  All calls on one GPU share the array:
 * calls that overlap on one GPU (several streams or threads) race and must be
 * serialised by the caller.  The first call on a device clears the array's
 * counters with a kernel on `stream`. */
size_t exl3_linear_noalloc_max_bytes(void);
int exl3_linear_forward_noalloc(const exl3_linear* handle, const void* x, int32_t x_type,
                                int64_t rows, void* y, int32_t y_type, void* stream);

/* Exl3Group::new/forward, linear.rs:2285-2382: up to 8 projections with the
 * same input width, K and codebook applied to one x (q/k/v, gate/up); ys[i]
 * receives parts[i]'s output in exl3_linear_output_dtype(parts[i], x_type)
 * (x's dtype; f32 for a biased member under bf16 activations).  One launch covers every member's
 * column blocks (rows <= 16), or one prologue launch and one QMM launch (rows
 * > 16); each member's output is bit-identical to its own exl3_linear_forward.
 * Workspace: exl3_group_workspace_bytes. */
size_t exl3_group_workspace_bytes(const exl3_linear* const* parts, int32_t count, int64_t rows);
int exl3_group_forward(const exl3_linear* const* parts, int32_t count, const void* x,
                       int32_t x_type, int64_t rows, void* const* ys, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Array::swiglu, native/ffi/mlx_bridge.cpp:745-749: out[i] =
 * (g * sigmoid(g)) * u of f16 gate[i], up[i], every operation rounded to f16
 * (sigmoid as MLX: y = 1 / (1 + exp(-|g|)), g < 0 ? 1 - y : y). */
int exl3_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t count,
                void* stream);

/* Array::geglu, native/ffi/mlx_bridge.cpp:764-774: out[i] =
 * (0.5g * (1 + tanh(0.7978845608 * (g + 0.044715 * g^3)))) * u of f16
 * gate[i], up[i] with f16 constants, every operation rounded to f16 (pow and
 * tanh rounded once from their binary64 values). */
int exl3_geglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t count,
               void* stream);

/* Dense SwiGLU MLP of a decoder layer, qwen35.rs:303-307 (Exl3Group of
 * gate/up, Array::swiglu, down Exl3Linear::forward): y[rows][down.out] =
 * down(swiglu(gate(x), up(x))), f16 x and y; gate and up share in, out, K and
 * codebook, down.in = gate.out.  The SwiGLU (and, for rows > 16, the down
 * projection's input prologue) runs in the epilogue of the (gate, up) launch;
 * the result is bit-identical to exl3_group_forward + exl3_swiglu +
 * exl3_linear_forward.  Workspace: exl3_mlp_workspace_bytes. */
size_t exl3_mlp_workspace_bytes(const exl3_linear* gate, const exl3_linear* up,
                                const exl3_linear* down, int64_t rows);
int exl3_mlp_forward(const exl3_linear* gate, const exl3_linear* up, const exl3_linear* down,
                     const uint16_t* x, int64_t rows, uint16_t* y, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Exl3SwitchGlu::new, moe.rs:809-900 (SiLU).  gu_trellis
 * [in/16][2*E*H/16][16k] (gate tiles of expert e at columns [e*H/16,
 * (e+1)*H/16), up tiles at [(E+e)*H/16, ...), moe.rs:756-760); gu_suh
 * f16[E][2][in]; gu_svh f16[E][2][H]; down_trellis [H/16][E*in/16][16k];
 * down_suh f16[E][H]; down_svh f16[E][in]. */
int exl3_moe_create(const uint16_t* gu_trellis, const uint16_t* gu_suh, const uint16_t* gu_svh,
                    const uint16_t* down_trellis, const uint16_t* down_suh,
                    const uint16_t* down_svh, int32_t in, int32_t hidden, int32_t experts,
                    int32_t top_k, int32_t k, int32_t cb, exl3_moe** out_handle);
/* Exl3SwitchGlu::new_with_activation with GluActivation::Gelu (moe.rs:838-903,
 * as from_gemma_checkpoint builds it, :663-680): the same bank layout;
 * exl3_moe_forward then follows forward_gelu (moe.rs:1087-1153) -- gate and up
 * as the linear's outputs (staged Hadamard, *svh), Array::geglu, GEGLU
 * outputs of columns >= logical_hidden set to zero, the down projection's
 * input prepared as the linear's prologue.  logical_hidden >= hidden zeroes
 * nothing; logical_hidden <= 0 is rejected. */
int exl3_moe_create_gelu(const uint16_t* gu_trellis, const uint16_t* gu_suh,
                         const uint16_t* gu_svh, const uint16_t* down_trellis,
                         const uint16_t* down_suh, const uint16_t* down_svh, int32_t in,
                         int32_t hidden, int32_t experts, int32_t top_k, int32_t k, int32_t cb,
                         int32_t logical_hidden, exl3_moe** out_handle);
void exl3_moe_destroy(exl3_moe* handle);
/* Input width and per-expert hidden width of a SwitchGLU handle (the
 * reference's Exl3SwitchGlu input / hidden fields, moe.rs:886-896); 0 for a
 * null handle. */
int32_t exl3_moe_in_features(const exl3_moe* handle);
int32_t exl3_moe_hidden_features(const exl3_moe* handle);
size_t exl3_moe_workspace_bytes(const exl3_moe* handle, int64_t rows);

/* Exl3SwitchGlu::forward, moe.rs:905-975: x [rows][in] of x_type (f16, bf16
 * or f32; cast to f16 before the input scales, as routed_inputs reads
 * half(x), moe.rs:205-206), selected u32[rows][top_k] (< experts), scores
 * [rows][top_k] of scores_type.  y [rows][in] in the dtype of the reference's
 * weighted sum (finish_and_reduce, moe.rs:602-608: f16 expert outputs times
 * the scores, summed over top_k): f16 for f16 scores (f16 products, f32 sum
 * rounded to f16); f32 for f32 or bf16 scores (MLX promotes f16 * f32 and
 * f16 * bf16 to f32: f32 products and sum).  The routing plan (moe.rs:66-182)
 * is built on the device. */
int exl3_moe_forward(const exl3_moe* handle, const void* x, int32_t x_type, int64_t rows,
                     const uint32_t* selected, const void* scores, int32_t scores_type, void* y,
                     void* workspace, size_t workspace_bytes, void* stream);

/* The mapped expert QMV, expert_mapped (linear.rs:2817-2852; its layout,
 * expert_mapped_layout :3054-3336, for a route-major bank): x [rows][in] of
 * x_type (f16, bf16 or f32) with rows = routes * projections, per-row input
 * scales suh [rows][in] f16, a bank trellis [in/16][bank_tiles][16k] u16 and
 * routes selected u32[routes].  Row r = route * projections + p multiplies
 * tile columns selected[route] * out/16 + p * stride_tiles + t (t < out/16)
 * by xhat_r = f16(H128(f16(f16(x_r) * suh_r)) / sqrt(128)).  raw != 0: y is
 * the f32 product [rows][out] (svh unused, may be NULL); else y [rows][out] of
 * x_type is f16(H128(f16(yhat)) / sqrt(128)) * svh_r (svh [rows][out] f16)
 * cast to x's dtype.  Checks as expert_mapped_layout, plus a 128-aligned
 * input and every projection's columns inside the bank; rows whose expert
 * index leaves the bank (device data) produce zeros.  Rows are independent
 * of each other (the K-split depends on `in` only). */
size_t exl3_expert_mapped_workspace_bytes(int32_t in, int32_t out, int64_t rows);
int exl3_expert_mapped(const uint16_t* trellis, int32_t in, int32_t bank_tiles, int32_t k,
                       int32_t cb, const void* x, int32_t x_type, int64_t rows,
                       const uint16_t* suh, const uint32_t* selected, int32_t routes,
                       int32_t projections, int32_t out, int32_t stride_tiles,
                       const uint16_t* svh, int32_t raw, void* y, void* workspace,
                       size_t workspace_bytes, void* stream);

/* The input prologue of every EXL3 projection as an op of its own,
 * exl3_prepare128 (exl3.metal:204-216; the `metal-prepare128` codec op,
 * main.rs:1338-1342, gpu.rs:1537-1558): out[i] = f16(H128(f16(x[i] * s)) /
 * sqrt(128)) over consecutive 128-element blocks of f16 rows of `width`
 * elements, with the Hadamard's f16 staging, s = scales[i % width]
 * (scale_count == width) or scales[i] (scale_count == elements).  Rejects, as
 * prepare128_blocks (contracts.rs:2146-2159), widths that are not positive
 * multiples of 128, incomplete rows, other scale counts and more than 2^32 - 1
 * elements; zero elements is a no-op. */
int exl3_prepare128(const uint16_t* x, int64_t elements, int32_t width, const uint16_t* scales,
                    int64_t scale_count, uint16_t* out, void* stream);

/* The SwitchGLU glue steps as ops of their own (the exl3_moe_forward
 * epilogues compute the same per slot):
 * swiglu_down_input (moe.rs:569-583, glu_down_input :435-563 with SiLU):
 * gate_up f32 [slots*2][hidden] (gate row 2s, up row 2s+1), gu_svh f16
 * [experts][2][hidden], down_suh f16 [experts][hidden], selected u32 [slots]
 * -> xhat f16 [slots][hidden], the down projection's input (slots routed to
 * ids >= experts get zeros).  finish_and_reduce (moe.rs:586-609): raw f32
 * [rows*top_k][width], svh f16 [rows*top_k][width], scores [rows][top_k] of
 * scores_type -> y [rows][width], f16 for f16 scores and f32 for f32 or bf16
 * scores (the promotion of exl3_moe_forward). */
int exl3_swiglu_down_input(const float* gate_up, const uint16_t* gu_svh, const uint16_t* down_suh,
                           const uint32_t* selected, int64_t slots, int32_t hidden,
                           int32_t experts, uint16_t* xhat, void* stream);
int exl3_finish_and_reduce(const float* raw, const uint16_t* svh, const void* scores,
                           int32_t scores_type, int64_t rows, int32_t top_k, int32_t width,
                           void* y, void* stream);

/* Decode hook, the reference's `metal-decode` codec op (exl3.metal:102-109,
 * main.rs:945-967): for every tile, states[t*256 + i] (nullable) and the f16
 * bits values[t*256 + i] of state index i, in the tile's stored order. */
int exl3_decode_tiles(const uint16_t* packed, int64_t tiles, int32_t k, int32_t cb,
                      uint16_t* states, uint16_t* values, void* stream);

/* Packing hook, the reference's `metal-pack` codec op (exl3_pack,
 * exl3.metal:85-100; codec::pack, codec.rs:73-100): packed[t*16k + i] = the
 * trellis tile of the low k bits of states[t*256 .. +255], the inverse of
 * exl3_decode_tiles' states. */
int exl3_pack_tiles(const uint16_t* states, int64_t tiles, int32_t k, uint16_t* packed,
                    void* stream);

/* Codewords of arbitrary states, the `codebook` codec op (main.rs:301-307,
 * decode_codeword codec.rs:52-71): values[i] = f16 bits of codeword(states[i]). */
int exl3_codewords(const uint16_t* states, int64_t count, int32_t cb, uint16_t* values,
                   void* stream);

/* The reference's serial inner QMV without glue, the `metal-qmv` codec op
 * (gpu.rs:1561-1593 with exl3_qmv, exl3.metal:118-142): y[n] =
 * f16(sum_r x[r] * W[r][n]) for a packed trellis of rows x cols (both
 * multiples of 16) in [rows/16][cols/16][16k] order, x f16[rows], y f16[cols];
 * f32 accumulation.  Workspace: exl3_qmv_inner_workspace_bytes (the decoded
 * tiles). */
size_t exl3_qmv_inner_workspace_bytes(int32_t rows, int32_t cols);
int exl3_qmv_inner(const uint16_t* packed, int32_t rows, int32_t cols, int32_t k, int32_t cb,
                   const uint16_t* x, uint16_t* y, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Fault hook for tests and harnesses (no counterpart in the reference; it
 * plays the part of a failing Metal launch under protect(),
 * mlx_bridge.cpp:56-66): every later launch whose name contains `text` fails
 * with EXL3_EDEVICE and "<name>: forced launch failure" -- the entry points'
 * first launches before anything is issued (nothing written, usable without a
 * GPU), later ones after issuing (the kernels that write the output are then
 * never launched, and the workspace stays valid for the next call).  NULL
 * disarms.  EXL3_FAIL_LAUNCH in the environment arms it at load. */
void exl3_debug_fail_launch(const char* text);

/* ------------------------------------------------------------------------
 * Checkpoints (safetensors EXL3 model directories).
 *
 * exl3_checkpoint_open replaces checkpoint::inspect
 * (native/src/checkpoint.rs:197-330, with read_header :38-93): it reads
 * config.json, quantization_config.json (quant_method "exl3",
 * tensor_storage) and the header of every model*.safetensors shard, and
 * validates them with the reference's checks and messages (payload tiled by
 * the tensors exactly, no duplicate tensors, tokenizer files present,
 * stored_tensors shapes, every exl3 module's trellis and suh/svh (or legacy
 * su/sv), the shard index).  No payload is read; shards stay open until
 * exl3_checkpoint_close.  A checkpoint handle is immutable and may be shared
 * between threads.
 * ------------------------------------------------------------------------ */
typedef struct exl3_checkpoint exl3_checkpoint;

/* TensorInfo (checkpoint.rs:15-26) of one tensor. */
typedef struct {
  char dtype[8];      /* safetensors dtype, e.g. "I16", "F16" */
  int32_t ndim;       /* at most 8 */
  int64_t shape[8];
  uint64_t offset;    /* absolute byte offset of the payload in its shard */
  uint64_t bytes;     /* payload size */
  const char* shard;  /* shard path, valid until the checkpoint is closed */
} exl3_tensor_info;

int exl3_checkpoint_open(const char* dir, exl3_checkpoint** out_handle);
void exl3_checkpoint_close(exl3_checkpoint* ckpt);

/* Checkpoint fields (checkpoint.rs:129-137): canonical path, config
 * model_type ("unknown" if absent), quantization bits (NaN if absent), total
 * size of the directory's files, sorted exl3 module prefixes. */
const char* exl3_checkpoint_path(const exl3_checkpoint* ckpt);
const char* exl3_checkpoint_model_type(const exl3_checkpoint* ckpt);
double exl3_checkpoint_bits(const exl3_checkpoint* ckpt);
uint64_t exl3_checkpoint_size_bytes(const exl3_checkpoint* ckpt);
int32_t exl3_checkpoint_module_count(const exl3_checkpoint* ckpt);
const char* exl3_checkpoint_module(const exl3_checkpoint* ckpt, int32_t index);

/* Tensor names in sorted order, and one tensor's record. */
int64_t exl3_checkpoint_tensor_count(const exl3_checkpoint* ckpt);
const char* exl3_checkpoint_tensor_name(const exl3_checkpoint* ckpt, int64_t index);
int exl3_checkpoint_tensor(const exl3_checkpoint* ckpt, const char* name, exl3_tensor_info* info);

/* TensorInfo::read_bytes (checkpoint.rs:113-125): copies the raw payload
 * into host memory `dst` of exactly info.bytes bytes. */
int exl3_checkpoint_read(const exl3_checkpoint* ckpt, const char* name, void* dst, size_t bytes);

/* A float tensor (F16, BF16 or F32) as `count` f16 values, rounded to nearest
 * even as MLX astype(Float16) rounds (the conversion exl3_linear_load applies
 * to scales and bias, linear.rs:527, :857, :993). */
int exl3_checkpoint_read_f16(const exl3_checkpoint* ckpt, const char* name, uint16_t* dst,
                             size_t count);

/* Exl3Linear::from_checkpoint (linear.rs:454-575): {prefix}.trellis (U16 or
 * I16), {prefix}.suh or .su, {prefix}.svh or .sv, optional {prefix}.bias;
 * codebook MUL1 if {prefix}.mul1 exists, else MCG if {prefix}.mcg exists,
 * else 3INST; K = last trellis dimension / 16.  Scales and bias are rounded
 * to f16 (F16, BF16 or F32 on disk).  The weights are uploaded to the current
 * HIP device; the handle owns them and exl3_linear_destroy frees them. */
int exl3_linear_load(const exl3_checkpoint* ckpt, const char* prefix, exl3_linear** out_handle);

/* Exl3SwitchGlu::from_checkpoint / from_lfm_checkpoint (moe.rs:629-660,
 * :681-800): experts {prefix}.{e}.{gate|up|down} for e < experts, projection
 * names "gate_proj"/"up_proj"/"down_proj" when NULL (LFM: "w1", "w3", "w2").
 * Every expert must share K, codebook and shapes; scales must be F16.  The
 * assembled bank is uploaded to the current HIP device and owned by the
 * handle. */
int exl3_moe_load(const exl3_checkpoint* ckpt, const char* prefix, int32_t experts, int32_t top_k,
                  const char* gate, const char* up, const char* down, exl3_moe** out_handle);

/* Exl3SwitchGlu::from_gemma_checkpoint (moe.rs:663-680): exl3_moe_load with
 * the gate_proj/up_proj/down_proj names, building a GELU bank as
 * exl3_moe_create_gelu does. */
int exl3_moe_load_gemma(const exl3_checkpoint* ckpt, const char* prefix, int32_t experts,
                        int32_t top_k, int32_t logical_hidden, exl3_moe** out_handle);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_HIP_H */
