// Launcher tables shared between the host translation unit and the kernel
// translation units (each kernel family is compiled in its own file so the
// instantiations over K x codebook build in parallel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_params.hpp"

struct exl3_linear;
struct exl3_moe;

namespace exl3 {

typedef void (*QmvFn)(const QmvParams&, dim3, size_t, hipStream_t);
typedef void (*QmmFn)(const QmmParams&, dim3, hipStream_t);
typedef void (*DecodeFn)(const uint32_t*, int64_t, uint16_t*, uint16_t*, dim3, hipStream_t);

// Every workspace starts with this many bytes of counters that are zero
// between calls; each entry point's scratch follows them.
constexpr size_t kWorkspaceCounterBytes = 65536;

// [K-1][codebook]
extern const QmvFn kQmv[3][8][3];  // [log2 KW]: 1, 2 or 4 K-parts per column pair
extern const QmvFn kQmvSingle[8][3];  // one row, one K-part per column pair
extern const QmvFn kQmvSingleShallow[8][3];  // the same with one slice per prefetch set
extern const QmvFn kQmvSingle2[8][3];  // one row, 2 K-parts per pair, shallow
extern const QmvFn kQmvFrag[8][3];    // one K-part per column pair, fragment-order partials
extern const QmvFn kQmvShallow[8][3];      // kQmv[0] with one slice per prefetch set
extern const QmvFn kQmvFragShallow[8][3];  // kQmvFrag with one slice per prefetch set
extern const DecodeFn kDecode[8][3];
extern const QmmFn kQmm[3][8][3];  // [log2 MB]: 64, 128 or 256 rows per workgroup

// xhat of `members` (suh, xhat) pairs of p in one launch.
void launch_prologue(const PrologueParams& p, int members, hipStream_t s);
// values[i] = codeword(states[i], cb).
void launch_codewords(const uint16_t* states, int64_t n, int cb, uint16_t* values, hipStream_t s);
// packed[t][16k] = the trellis tile of states[t][256] (low k bits of each).
void launch_pack_tiles(const uint16_t* states, int64_t tiles, int k, uint16_t* packed,
                       hipStream_t s);
// y = f16(x . W) over decoded tiles (no glue).
void launch_qmv_inner(const uint16_t* values, const uint16_t* x, int rows, int cols, uint16_t* y,
                      hipStream_t s);
// xhat = the down projection's prologue of swiglu(gate, up), [rows][H].
void launch_swiglu_prepare(const uint16_t* gate, const uint16_t* up, const uint16_t* down_suh,
                           int H, int rows, uint16_t* xhat, hipStream_t s);
// out[i] = swiglu(gate[i], up[i]) (Array::swiglu) or geglu(gate[i], up[i])
// (Array::geglu) in f16.
void launch_glu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, bool gelu,
                hipStream_t s);
void launch_fill_zero(uint32_t* p, size_t words, hipStream_t s);

// Records the thread-local error message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Converts a pending launch error into EXL3_EDEVICE (or the fault hook's
// forced failure for `what`, after the launch).
int check_launch(const char* what);
// The fault hook before a launch: EXL3_EDEVICE when `what` is armed.
int launch_gate(const char* what);

// Hands a device allocation (hipMalloc) to a handle, which frees it when it is
// destroyed: the checkpoint loaders own the weights they upload.
void adopt_device_memory(exl3_linear* h, void* mem);
void adopt_device_memory(exl3_moe* h, void* mem);

}  // namespace exl3

#define EXL3_CB_ROW(F, K) {F<K, 0>, F<K, 1>, F<K, 2>}
#define EXL3_TABLE(F)                                                              \
  {EXL3_CB_ROW(F, 1), EXL3_CB_ROW(F, 2), EXL3_CB_ROW(F, 3), EXL3_CB_ROW(F, 4), \
   EXL3_CB_ROW(F, 5), EXL3_CB_ROW(F, 6), EXL3_CB_ROW(F, 7), EXL3_CB_ROW(F, 8)}

// Explicit instantiation over K = 1..8 and the three codebooks, so both the
// device pass and the host pass see every kernel.
#define EXL3_INST_CB(M, K) M(K, 0) M(K, 1) M(K, 2)
#define EXL3_INSTANTIATE(M)                                                        \
  EXL3_INST_CB(M, 1) EXL3_INST_CB(M, 2) EXL3_INST_CB(M, 3) EXL3_INST_CB(M, 4) \
  EXL3_INST_CB(M, 5) EXL3_INST_CB(M, 6) EXL3_INST_CB(M, 7) EXL3_INST_CB(M, 8)
