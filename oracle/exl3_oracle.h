/*
 * CPU oracle for the EXL3 quantized-linear path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg are the only
 * callers.  The product library (mlxl3_amd/libexl3_hip.so) never links or
 * calls anything here.
 *
 * Every function restates the reference algorithm it names (file:line under
 * the reference tree) in plain C; f16/bf16 conversions are done bit-exactly by
 * hand so the oracle does not depend on compiler half-precision support.
 */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (IEEE binary16 / bfloat16, round-to-nearest-even) ---- */
float exl3o_f16_to_f32(uint16_t h);
uint16_t exl3o_f64_to_f16(double d);
uint16_t exl3o_f32_to_f16(float f);
float exl3o_bf16_to_f32(uint16_t h);
uint16_t exl3o_f32_to_bf16(float f);

/* ---- codec (native/src/codec.rs) ---- */
/* decode_codeword, codec.rs:52-71.  Returns f16 bits.  cb: 0 3INST, 1 MCG, 2 MUL1. */
uint16_t exl3o_codeword(uint16_t state, int cb);
/* codebook over all 65536 states (exhaustive table) */
void exl3o_codebook(int cb, uint16_t* out65536);
/* unpack, codec.rs:102-124 (+ unpack_window :40-46, packed_pair :48-50).
 * packed: tiles*16*k u16, states: tiles*256 u16.  Returns 0 or -1 (bad k). */
int exl3o_unpack(const uint16_t* packed, int64_t tiles, int k, uint16_t* states);
/* pack, codec.rs:73-100 (+ pack_source :34-38). */
int exl3o_pack(const uint16_t* states, int64_t tiles, int k, uint16_t* packed);
/* permutation, codec.rs:126-138: out[state index] = row*16 + col */
void exl3o_permutation(uint16_t out[256]);
/* reconstruct_inner, codec.rs:158-190: dense W_inner [rows][cols] f16 bits. */
int exl3o_reconstruct_inner(const uint16_t* packed, int k, int cb, int64_t rows,
                            int64_t cols, uint16_t* out);

/* ---- Hadamard-128 (in place over count values, count % 128 == 0) ---- */
/* MLX f32 hadamard_transform semantics: ascending-stride radix-2 butterflies
 * in f32, then * f32(1/sqrt(128)).  Pinned bit-exactly by the reference's
 * tests/fixtures/native-converter-host/hadamard.npz. */
void exl3o_h128_f32(float* v, int64_t count);
/* Engine f16 staging (exl3.metal:154-170, linear.rs:1380-1427): same
 * butterflies, values rounded to f16 after the stride-8 and stride-64 stages,
 * then f16(v * f32(1/sqrt(128))).  Values are returned as f32 holding f16. */
void exl3o_h128_staged(float* v, int64_t count);

/* Output dtype of a projection (linear.rs:992-995: y.astype(x.dtype) + the f16
 * bias under MLX's promotion): x_dtype, except DT_BF16 with a bias -> f32. */
int exl3o_result_dtype(int x_dtype, int has_bias);

/* ---- forward of one EXL3 linear ----
 * x: rows*in values of x_dtype (9 f16, 10 f32, 12 bf16), y: rows*out of
 * exl3o_result_dtype(x_dtype, bias != NULL).  trellis [in/16][out/16][16k] u16; suh [in] f16; svh [out] f16;
 * bias [out] f16 or NULL.
 * mode 0: ponyexl3/ref/forward.py:14-49 (f32 H128 with suh/svh in f32,
 *         f16 roundings at xh, y and the output) evaluated with f64 sums.
 * mode 1: engine glue semantics (linear.rs:847-865 prologue, :984-997
 *         epilogue): f16(x)*suh in f16, f16-staged H128, f32 GEMV, f16(y),
 *         f16-staged H128, *svh in f16, cast, + bias.
 * yhat_out (optional, rows*out f32): the raw inner product before rounding.
 * threads <= 0 uses all cores.  Returns 0 or a negative error. */
int exl3o_forward(int mode, const void* x, int x_dtype, int64_t rows, const uint16_t* trellis,
                  int in, int out, int k, int cb, const uint16_t* suh, const uint16_t* svh,
                  const uint16_t* bias, void* y, float* yhat_out, int threads);

/* xhat of the engine prologue (mode 1), rows*in f16 bits. */
int exl3o_prologue(const void* x, int x_dtype, int64_t rows, int in, const uint16_t* suh,
                   uint16_t* xhat);

/* ---- MoE SwitchGLU (moe.rs:66-609 semantics, one expert at a time) ----
 * gu_trellis [in/16][2*E*H/16][16k]: for expert e, gate columns are tile
 * columns [e*H/16, (e+1)*H/16) and up columns [(E+e)*H/16, ...) (moe.rs:756-760).
 * down_trellis [H/16][E*in/16][16k], expert e at tile columns [e*in/16, ...).
 * gu_suh [E][2][in], gu_svh [E][2][H], down_suh [E][H], down_svh [E][in] f16.
 * selected [rows][top_k] u32, scores [rows][top_k] of scores_dtype, x rows*in of
 * x_dtype (cast to f16 first, moe.rs:205-206).  y rows*in: f16 for f16 scores,
 * f32 for f32 or bf16 scores (finish_and_reduce's promotion, moe.rs:602-608).
 * Each routed slot: gate = lin(x), up = lin(x) (f16 outputs), act =
 * f16(silu(gate) * up), down = lin(act) (f16), y = sum_t score*down (f16
 * products and an f32 sum rounded to f16 for f16 scores; f32 otherwise).
 * gelu != 0: forward_gelu (moe.rs:1087-1153) -- gate/up and the down input
 * in the linear's engine glue (staged H128), act = geglu(gate, up) for
 * columns < logical_hidden and 0 beyond. */
/* expert_mapped (linear.rs:2817-2852, route-major bank): rows = routes *
 * projections rows of x (x_dtype) with per-row suh [rows][in] f16, bank
 * trellis [in/16][bank_tiles][16k], tile columns selected[route] * out/16 +
 * p * stride_tiles + t; raw: y f32 [rows][out]; else y [rows][out] of x_dtype
 * after the epilogue with per-row svh [rows][out].  Rows past the bank: 0. */
int exl3o_expert_mapped(const void* x, int x_dtype, int64_t rows, int in, const uint16_t* suh,
                        const uint16_t* trellis, int bank_tiles, int k, int cb,
                        const uint32_t* selected, int routes, int projections, int out,
                        int stride_tiles, const uint16_t* svh, int raw, void* y, int threads);

int exl3o_moe_forward(const void* x, int x_dtype, int64_t rows, int in, int hidden, int experts,
                      int top_k, int k, int cb, const uint16_t* gu_trellis,
                      const uint16_t* gu_suh, const uint16_t* gu_svh,
                      const uint16_t* down_trellis, const uint16_t* down_suh,
                      const uint16_t* down_svh, const uint32_t* selected, const void* scores,
                      int scores_dtype, void* y, int gelu, int logical_hidden, int threads);

/* glu_down_input with SiLU (moe.rs:435-583): gate_up f32 [slots*2][hidden]
 * (gate row 2s, up row 2s+1), gu_svh [E][2][hidden], down_suh [E][hidden],
 * selected [slots] -> xhat f16 [slots][hidden]. */
int exl3o_swiglu_down_input(const float* gate_up, const uint16_t* gu_svh,
                            const uint16_t* down_suh, const uint32_t* selected, int64_t slots,
                            int hidden, int experts, uint16_t* xhat);

/* finish_and_reduce (moe.rs:586-609): raw f32 [rows*top_k][width], svh f16
 * [rows*top_k][width], scores [rows][top_k] of scores_dtype -> y [rows][width],
 * f16 for f16 scores and f32 for f32 / bf16 scores. */
int exl3o_finish_and_reduce(const float* raw, const uint16_t* svh, const void* scores,
                            int scores_dtype, int64_t rows, int top_k, int width, void* y);

/* ---- dense SwiGLU (Array::swiglu, native/ffi/mlx_bridge.cpp:745-749) ----
 * out[i] = (g * sigmoid(g)) * u for f16 g, u in f16 arithmetic: the compiled
 * MLX expression evaluated on float16 arrays (MLX 0.32.2, the version the
 * engine pins), whose Sigmoid functor is y = 1 / (1 + exp(-|x|)),
 * x < 0 ? 1 - y : y.  Every operation rounds to f16; exp is evaluated in f32
 * (expf) and rounded. */
void exl3o_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n);

/* ---- dense GEGLU (Array::geglu, native/ffi/mlx_bridge.cpp:764-774) ----
 * out[i] = f16 evaluation of 0.5g(1 + tanh(0.7978845608(g + 0.044715g^3)))u:
 * every operation rounds to f16, pow(g, 3) and tanh are rounded once from
 * binary64. */
void exl3o_geglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
