// Kernel parameter blocks (plain structs passed by value to the kernels).
#pragma once

#include <stdint.h>

namespace exl3 {

// A launch covers up to kMaxMembers projections that share one input (a
// single linear is a group of one): their 128-column blocks are numbered
// consecutively, member i owning global blocks [cblk0, cblk0 + out/128).
constexpr int kMaxMembers = 8;

struct Member {
  const uint32_t* trellis;  // [in/16][out/16][8K] u32
  const uint16_t* suh;      // [in] f16 (QMV: fused prologue)
  const uint16_t* xhat;     // [M][in] f16 (QMM: prologue output of this member)
  const uint16_t* svh;      // [out] f16
  const uint16_t* bias;     // [out] f16 or null
  void* y;                  // [M][out] of y_dtype
  int out;                  // columns
  int cblk0;                // first global column block
  int y_dtype;              // x_dtype, or f32 for bf16 activations with a bias
};

// SwiGLU edge of a (gate, up) QMV group: members 0 and 1 have equal widths;
// the last workgroup to finish a 128-column block of both computes
// act = f16((g * sigmoid(g)) * u) for it and writes act [M][out] or, with
// down_suh set, the down projection's xhat [M][out]
// (f16(H128(f16(act * down_suh)) / sqrt(128))).
struct Glu {
  int on;
  uint16_t* out;             // act or down xhat, [M][out] f16
  const uint16_t* down_suh;  // null: write act
};

struct QmvParams {
  Member mem[kMaxMembers];
  int members;
  const void* x;       // [M][in] of x_dtype
  float* partials;     // [splits][M][total_out]
  uint32_t* counters;  // [total_out/128] (GLU: [out/128]), zero between calls
  int in, total_out, M, splits;
  int x_dtype;
  int prio_ramp;  // lower the waves' issue priority with progress (> 1 wave per SIMD)
  Glu glu;
};

struct QmmParams {
  Member mem[kMaxMembers];
  int members;
  float* partials;     // [splits][tiles][64*MB x 128 f32 in fragment order] (splits > 1)
  uint32_t* counters;  // [mtiles * col_blocks], zero between calls (splits > 1)
  int in, total_out, M;
  int x_dtype;         // the activation dtype (the output's intermediate cast)
  int col_blocks;      // total_out / 128
  int mtiles;          // ceil(M / rows per workgroup)
  int splits;          // K-ranges per output tile (global split-K)
};

struct PrologueParams {
  const void* x;  // [rows][in] of x_dtype
  int x_dtype, in, rows;
  const uint16_t* suh[kMaxMembers];
  uint16_t* xhat[kMaxMembers];  // [rows][in] f16 each
  size_t suh_stride;            // scale elements per row: 0 (one scale per column) or in
};

// The member owning global column block `cblk`, chosen with compile-time
// indices only (a dynamically indexed parameter array would be copied to
// scratch memory).
template <typename P>
__device__ __forceinline__ Member select_member(const P& p, int cblk) {
  Member m = p.mem[0];
#pragma unroll
  for (int i = 1; i < kMaxMembers; ++i)
    if (i < p.members && cblk >= p.mem[i].cblk0) m = p.mem[i];
  return m;
}

}  // namespace exl3
