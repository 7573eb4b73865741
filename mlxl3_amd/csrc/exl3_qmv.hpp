// Kernels for the EXL3 linear at M <= 16 rows (batch-1 decode and the small
// speculative-verify batches): the QMV family of the reference
// (_qmv_tile_kernel.metal, dispatched from linear.rs:866-960 and
// forward_qmv_batch linear.rs:1024-1216), re-designed for gfx950.
//
// One launch does the whole linear:
//   1. prologue (linear.rs:847-865): the workgroup computes
//      xhat = f16(H128(f16(x) * suh) / sqrt(128)) for its K-split's input rows
//      straight into LDS (the trellis loads for the first tiles are already in
//      flight);
//   2. the weight stream: each wave owns two adjacent output tiles (32
//      columns) and walks its K-split four tile-rows at a time; one 64-lane
//      K-dword load brings in 8 whole tiles (lanes 16g..16g+15 hold tile row
//      tk0+g, tiles tn0 and tn0+1).  Lanes decode their 32 weights in
//      registers into MFMA B fragments and v_mfma_f32_16x16x32_f16 multiplies
//      them with up to 16 activation rows at once (rows >= M repeat row M-1
//      and are never stored), so M = 1..16 costs the same decode;
//   3. split-K partials go to the workspace (row-major, or in fragment order
//      from 8 rows); the last workgroup to finish a 128-column block sums the
//      splits in split order (deterministic), and applies the epilogue
//      (linear.rs:984-997): f16, H128, * svh, cast, bias.
#pragma once

#include "exl3_device.hpp"
#include "exl3_params.hpp"

namespace exl3 {

// Phase stamps of the single-row QMV, compiled only into the phase-probe build
// of the library (-DEXL3_QMV_PHASES; mlxl3_amd/phases.py drives it).  While
// qmv_phase_out is set, every wave of a single-row launch writes kPhaseWords
// words at qmv_phase_out[(workgroup * waves + wave) * kPhaseWords]: the
// 100 MHz realtime counter at entry, at the loop start and end, at its
// counter arrival and at the end of the epilogue (last arrivers), the shader
// clock at the loop start and end, and HW_ID | XCC_ID << 32 | last << 48.
#ifdef EXL3_QMV_PHASES
static __device__ unsigned long long* qmv_phase_out;
constexpr int kPhaseWords = 8;
#define EXL3_PHASE(stmt) stmt
#else
#define EXL3_PHASE(stmt)
#endif

// Slices per prefetch set of the mapped-expert weight stream (two sets in
// flight).
template <int K>
constexpr int kQmvDepth = K <= 4 ? 4 : 2;
// Slices per prefetch set of the QMV weight loop (two sets in flight).  With
// the loop branch-free and the slices buffer loads, shallower sets won (same
// box, K=4: NS 14.23 -> 13.65 us with 2 instead of 4, 14.8 us with 1; K=5:
// 24.97 -> 24.41 us with 1 instead of 2).
template <int K>
constexpr int kQmvLoopDepth = K <= 4 ? 2 : 1;

// Split-K sums load this many splits' partials together.
constexpr int kSplitChunk = 8;

// Split-K partials cross workgroups (and XCDs): agent-scope relaxed atomics.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// v0 += sum over splits s of col[s * stride + lane], v1 likewise at lane + 64,
// added in split order.  Coherent loads are served one after another (~50 ns
// each, measured), so exactly `splits` of them are issued per column, up to
// kSplitChunk splits in flight at a time.
template <int C>
__device__ __forceinline__ void sum_split_chunk(const float* col, size_t stride, int s0, int lane,
                                                float& v0, float& v1) {
  float a[C], b[C];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const float* ps = col + (size_t)(s0 + i) * stride;
    a[i] = load_coherent(ps + lane);
    b[i] = load_coherent(ps + lane + 64);
  }
#pragma unroll
  for (int i = 0; i < C; ++i) {
    v0 += a[i];
    v1 += b[i];
  }
}
__device__ __forceinline__ void sum_split_columns(const float* col, size_t stride, int splits,
                                                  int lane, float& v0, float& v1) {
  int s0 = 0;
  for (; s0 + kSplitChunk <= splits; s0 += kSplitChunk)
    sum_split_chunk<kSplitChunk>(col, stride, s0, lane, v0, v1);
  switch (splits - s0) {
    case 7: sum_split_chunk<7>(col, stride, s0, lane, v0, v1); break;
    case 6: sum_split_chunk<6>(col, stride, s0, lane, v0, v1); break;
    case 5: sum_split_chunk<5>(col, stride, s0, lane, v0, v1); break;
    case 4: sum_split_chunk<4>(col, stride, s0, lane, v0, v1); break;
    case 3: sum_split_chunk<3>(col, stride, s0, lane, v0, v1); break;
    case 2: sum_split_chunk<2>(col, stride, s0, lane, v0, v1); break;
    case 1: sum_split_chunk<1>(col, stride, s0, lane, v0, v1); break;
    default: break;
  }
}

// Load the previous lane's last word of the same tile (word j*K-1, wrapping to
// the tile's last word for j == 0) and then the K words of this lane's slice
// of a tile: w[0] = previous word, w[1..K] = own words.  `p` points at the
// lane's own words; `prev_off` is -1 or 8K-1.
template <int K>
__device__ __forceinline__ void load_slice_prev(const uint32_t* __restrict__ p, int prev_off,
                                                uint32_t (&w)[K + 1]) {
  w[0] = __builtin_nontemporal_load(p + prev_off);
  if constexpr (K == 4) {
    u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    w[1] = v[0], w[2] = v[1], w[3] = v[2], w[4] = v[3];
  } else if constexpr (K == 8) {
    u32x4 v0 = __builtin_nontemporal_load((const u32x4*)p);
    u32x4 v1 = __builtin_nontemporal_load((const u32x4*)p + 1);
    w[1] = v0[0], w[2] = v0[1], w[3] = v0[2], w[4] = v0[3];
    w[5] = v1[0], w[6] = v1[1], w[7] = v1[2], w[8] = v1[3];
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) w[i + 1] = __builtin_nontemporal_load(p + i);
  }
}

// The same loads as raw buffer loads: the resource holds a workgroup-uniform
// base, `soff` the slice's scalar byte offset, `loff` / `loff_prev` the lane's
// byte offsets (its own words, the previous lane's last word), so a slice costs
// no vector address arithmetic and every access is bounded by the resource.
template <int K>
__device__ __forceinline__ void load_slice_prev_b(__amdgpu_buffer_rsrc_t w, uint32_t soff,
                                                  uint32_t loff, uint32_t loff_prev,
                                                  uint32_t (&out)[K + 1]) {
  out[0] = __builtin_amdgcn_raw_buffer_load_b32(w, loff_prev, soff, kCpolNt);
  if constexpr (K == 4 || K == 8) {
#pragma unroll
    for (int h = 0; h < K / 4; ++h) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(w, loff + 16 * h, soff, kCpolNt);
      out[4 * h + 1] = v[0], out[4 * h + 2] = v[1], out[4 * h + 3] = v[2], out[4 * h + 4] = v[3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i)
      out[i + 1] = __builtin_amdgcn_raw_buffer_load_b32(w, loff + 4 * i, soff, kCpolNt);
  }
}

// Decode the 4 B fragments of one 8-tile load and run the 4 MFMAs.  B[0] is
// the previous lane's last word of the same tile, B[1..K] the lane's words.
template <int K, int CB>
__device__ __forceinline__ void qmv_step_prev(const uint32_t (&B)[K + 1], half8 a0, half8 a1,
                                              float4v& acc0, float4v& acc1) {
  uint32_t src[32];
  extract_states<K>(B, src);
  half8 b00 = decode_fragment<CB, K, 0, 0>(src);
  half8 b01 = decode_fragment<CB, K, 0, 1>(src);
  mfma_operand_fence(b00, b01);
  acc0 = mfma16(a0, b00, acc0);
  acc1 = mfma16(a0, b01, acc1);
  half8 b10 = decode_fragment<CB, K, 1, 0>(src);
  half8 b11 = decode_fragment<CB, K, 1, 1>(src);
  mfma_operand_fence(b10, b11);
  acc0 = mfma16(a1, b10, acc0);
  acc1 = mfma16(a1, b11, acc1);
}

// qmv_step_prev in two halves: the decode of a step's 4 B fragments, and
// their 4 MFMAs (in the same order).
template <int K, int CB>
__device__ __forceinline__ void decode_step(const uint32_t (&B)[K + 1], half8 (&b)[4]) {
  uint32_t src[32];
  extract_states<K>(B, src);
  b[0] = decode_fragment<CB, K, 0, 0>(src);
  b[1] = decode_fragment<CB, K, 0, 1>(src);
  b[2] = decode_fragment<CB, K, 1, 0>(src);
  b[3] = decode_fragment<CB, K, 1, 1>(src);
  mfma_operand_fence(b[0], b[1]);
  mfma_operand_fence(b[2], b[3]);
}
__device__ __forceinline__ void mma_step(half8 a0, half8 a1, const half8 (&b)[4], float4v& acc0,
                                         float4v& acc1) {
  acc0 = mfma16(a0, b[0], acc0);
  acc1 = mfma16(a0, b[1], acc1);
  acc0 = mfma16(a1, b[2], acc0);
  acc1 = mfma16(a1, b[3], acc1);
}

// Epilogue for one row of a 128-column block held as (v0, v1) = columns
// (lane, lane+64): f16(sum) -> staged H128 -> f16(*1/sqrt128) -> f16(*svh)
// (finish_vals128), then cast (+bias) and store (finish_row128).
__device__ __forceinline__ void finish_vals128(float& v0, float& v1, int lane, int col0,
                                               const uint16_t* __restrict__ svh) {
  v0 = round_f16(v0);
  v1 = round_f16(v1);
  h128_wave<true>(v0, v1, lane);
  v0 = round_f16(v0 * kHadScale);
  v1 = round_f16(v1 * kHadScale);
  v0 = round_f16(v0 * h2f(svh[col0 + lane]));
  v1 = round_f16(v1 * h2f(svh[col0 + lane + 64]));
}
__device__ __forceinline__ void finish_row128(float v0, float v1, int lane, int col0,
                                              const uint16_t* __restrict__ svh,
                                              const uint16_t* __restrict__ bias, void* y,
                                              int y_dtype, int x_dtype, size_t row_off) {
  finish_vals128(v0, v1, lane, col0, svh);
  int c0 = col0 + lane, c1 = col0 + lane + 64;
  store_out(y, y_dtype, x_dtype, row_off + c0, v0, bias, c0);
  store_out(y, y_dtype, x_dtype, row_off + c1, v1, bias, c1);
}
// f16 output value with the optional bias added in f16 (y + bias).
__device__ __forceinline__ float with_bias_f16(float v16, const uint16_t* __restrict__ bias,
                                               int col) {
  return bias ? round_f16(v16 + h2f(bias[col])) : v16;
}

// SwiGLU of f16 operands in f16 arithmetic, the compiled MLX expression
// (g * sigmoid(g)) * u of Array::swiglu (native/ffi/mlx_bridge.cpp:745-749),
// with MLX's sigmoid y = 1 / (1 + exp(-|g|)), g < 0 ? 1 - y : y; every
// operation rounds to f16 (exp is evaluated in f32 and rounded).
__device__ __forceinline__ float sigmoid_f16(float g) {
  const float e = round_f16(expf(-fabsf(g)));
  const float y = round_f16(1.0f / round_f16(1.0f + e));
  return g < 0.f ? round_f16(1.0f - y) : y;
}
__device__ __forceinline__ float swiglu_f16(float g, float u) {
  return round_f16(round_f16(g * sigmoid_f16(g)) * u);
}

// binary64 -> binary16 rounded once to nearest even: round to odd into
// binary32 (24 >= 11 + 2 bits, so the nearest-even binary32 -> binary16 step
// that follows cannot round twice).
__device__ __forceinline__ float round_f16_f64(double d) {
  float f = (float)d;
  if ((double)f != d) {
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    if (!(b & 1u)) b = fabs((double)f) > fabs(d) ? b - 1u : b + 1u;  // the odd neighbour
    f = __builtin_bit_cast(float, b);
  }
  return round_f16(f);
}

// GEGLU of f16 operands in f16 arithmetic, the compiled MLX expression of
// Array::geglu (native/ffi/mlx_bridge.cpp:764-774):
// (0.5g * (1 + tanh(0.7978845608 * (g + 0.044715 * g^3)))) * u with f16
// constants; every operation rounds to f16, pow(g, 3) (exact in binary64) and
// tanh are rounded once from binary64.
__device__ __forceinline__ float geglu_f16(float g, float u) {
  const double gd = g;
  const float cube = round_f16_f64(gd * gd * gd);
  const float t = round_f16(g + round_f16(round_f16(0.044715f) * cube));
  const float inner = round_f16(round_f16(0.7978845608028654f) * t);
  const float th = round_f16_f64(tanh((double)inner));
  const float gelu = round_f16(round_f16(0.5f * g) * round_f16(1.0f + th));
  return round_f16(gelu * u);
}

// Prologue for one row of one 128-input block, split into its loads and its
// arithmetic so callers can put other memory traffic between the two:
// xhat = f16(H128(f16(f16(x) * suh)) / sqrt(128)) for elements (lane, lane+64).
struct PrologueIn {
  uint32_t x0lo, x0hi, x1lo, x1hi;  // raw 16-bit halves of the two activations
  uint32_t s0, s1;                  // raw suh bits (f16)
};
// Raw 16-bit loads only (the high half of an f32 is a second load, issued
// for f32 activations only, under a uniform branch); the loads stay in flight
// until prologue_finish consumes them.
__device__ __forceinline__ PrologueIn prologue_load(const void* x, int x_dtype, size_t off,
                                                    const uint16_t* __restrict__ suh, int e0,
                                                    int lane) {
  const uint16_t* xb = (const uint16_t*)x;
  const bool f32 = x_dtype == DT_F32;
  const size_t esz = f32 ? 2 : 1;  // u16 words per element
  const size_t i0 = (off + lane) * esz, i1 = (off + lane + 64) * esz;
  PrologueIn in;
  in.x0lo = xb[i0];
  in.x1lo = xb[i1];
  in.x0hi = in.x1hi = 0u;
  if (f32) {
    in.x0hi = xb[i0 + 1];
    in.x1hi = xb[i1 + 1];
  }
  in.s0 = suh[e0 + lane];
  in.s1 = suh[e0 + lane + 64];
  return in;
}
__device__ __forceinline__ float raw_act(uint32_t bits, int x_dtype) {
  if (x_dtype == DT_F32) return __builtin_bit_cast(float, bits);
  if (x_dtype == DT_BF16) return bf2f((uint16_t)bits);
  return h2f((uint16_t)bits);
}
__device__ __forceinline__ void prologue_finish(const PrologueIn& in, int x_dtype, int lane,
                                                float& v0, float& v1) {
  const uint32_t x0 = in.x0lo | (in.x0hi << 16), x1 = in.x1lo | (in.x1hi << 16);
  v0 = round_f16(round_f16(raw_act(x0, x_dtype)) * h2f((uint16_t)in.s0));
  v1 = round_f16(round_f16(raw_act(x1, x_dtype)) * h2f((uint16_t)in.s1));
  h128_wave<true>(v0, v1, lane);
  v0 = round_f16(v0 * kHadScale);
  v1 = round_f16(v1 * kHadScale);
}

// Prologue in the pair layout (lane holds elements 2*lane and 2*lane+1 of a
// 128-input block): one 32-bit (64-bit for f32) activation load and one 32-bit
// suh load per lane.  The butterflies run in the same ascending order with the
// same roundings as h128_wave: stride 1 inside the lane, strides 2..64 across
// lanes 1..32, f16 rounding after strides 8 and 64.
template <int STRIDE>
__device__ __forceinline__ float bfly_lane(float v, int lane) {
  float p = xor_lanes<STRIDE>(v);
  return (lane & STRIDE) ? p - v : v + p;
}

// Staged Hadamard-128 of a block held as 8 consecutive elements per lane, 16
// lanes per block (a DPP row): element strides 1, 2, 4 inside the lane, 8..64
// across lanes 1..8, f16 rounding after strides 8 and 64 (the reference's
// radix staging: strides in increasing order, f32 between the roundings).
__device__ __forceinline__ void h128_lane8(float (&v)[8], int lane) {
#pragma unroll
  for (int s = 1; s < 8; s <<= 1)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (!(j & s)) {
        const float a0 = v[j], b0 = v[j + s];
        v[j] = a0 + b0;
        v[j + s] = a0 - b0;
      }
  // stride 8 = lane bit 0, then f16 rounding
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = round_f16(bfly_lane<1>(v[j], lane));
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[j] = bfly_lane<2>(v[j], lane);  // stride 16
    v[j] = bfly_lane<4>(v[j], lane);  // stride 32
    v[j] = round_f16(bfly_lane<8>(v[j], lane));  // stride 64
  }
}

// Tail of prologue8: dst[0..7] = f16(H128(f16(f16(a) * s)) / sqrt(128)) over
// the row of 16 lanes (stored only if live).
template <bool VEC>
__device__ __forceinline__ void finish8_scaled(float (&v)[8], uint16_t* dst, bool live, int lane) {
  h128_lane8(v, lane);
  if (!live) return;
  if constexpr (VEC) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = (uint32_t)f2h(v[2 * i] * kHadScale) | ((uint32_t)f2h(v[2 * i + 1] * kHadScale) << 16);
    *(u32x4*)dst = o;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = f2h(v[i] * kHadScale);
  }
}
template <bool VEC>
__device__ __forceinline__ void finish8(const float (&a)[8], const float (&sv)[8], uint16_t* dst,
                                        bool live, int lane) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = round_f16(round_f16(a[i]) * sv[i]);
  finish8_scaled<VEC>(v, dst, live, lane);
}

// The activation inputs of prologue8: a[i] = x[xe + i] (f16, bf16 or f32),
// with 16-byte loads under VEC.
template <bool VEC>
__device__ __forceinline__ void load8_act(const void* x, int x_dtype, size_t xe, float (&a)[8]) {
  if constexpr (VEC) {
    if (x_dtype == DT_F32) {
      const float4v* xp = (const float4v*)((const float*)x + xe);
      const float4v x0 = xp[0], x1 = xp[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = x0[i];
        a[i + 4] = x1[i];
      }
    } else {
      const u32x4 xw = *(const u32x4*)((const uint16_t*)x + xe);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[2 * i] = raw_act(xw[i] & 0xffffu, x_dtype);
        a[2 * i + 1] = raw_act(xw[i] >> 16, x_dtype);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      a[i] = x_dtype == DT_F32 ? ((const float*)x)[xe + i]
                               : raw_act(((const uint16_t*)x)[xe + i], x_dtype);
  }
}

// The scale inputs of prologue8: sv[i] = sp[i] (f16).
template <bool VEC>
__device__ __forceinline__ void load8_scale(const uint16_t* sp, float (&sv)[8]) {
  if constexpr (VEC) {
    const u32x4 sw = *(const u32x4*)sp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[2 * i] = h2f((uint16_t)sw[i]);
      sv[2 * i + 1] = h2f((uint16_t)(sw[i] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) sv[i] = h2f(sp[i]);
  }
}

template <bool VEC>
__device__ __forceinline__ void load8(const void* x, int x_dtype, size_t xe, const uint16_t* sp,
                                      float (&a)[8], float (&sv)[8]) {
  load8_act<VEC>(x, x_dtype, xe, a);
  load8_scale<VEC>(sp, sv);
}

// f16(H128(f16(f16(x) * suh)) / sqrt(128)) of one 128-input block, held as
// 8 consecutive inputs per lane and 16 lanes (one DPP row) per block: x[xe..]
// and sp[0..7] are the lane's inputs and scales, dst[0..7] its xhat.  The
// whole Hadamard runs on DPP exchanges inside the row, and every lane moves
// 16-byte words (VEC; callers whose x, scales or output are not 16-byte
// aligned take the element-wise loads instead).  All 16 lanes of the row
// must be active; `live` = false computes without storing.
// v[i] = f16(x[i] * s[i]) for 8 f16 activations and scales held as raw
// 16-byte words, as packed f16 products.  Equal to round_f16(round_f16(a) * s)
// of finish8: the f32 product of two f16 values is exact (11-bit
// significands, at least 2^-48), so its one rounding to f16 is the IEEE f16
// product.  Each element is copied to a scalar before the bit cast (this
// hipcc casts element 0 for every v[i] of an ext-vector operand).
__device__ __forceinline__ void scale8_f16(const u32x4 xw, const u32x4 sw, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t xi = xw[i], si = sw[i];
    const half2v q = __builtin_bit_cast(half2v, xi) * __builtin_bit_cast(half2v, si);
    v[2 * i] = (float)q[0];
    v[2 * i + 1] = (float)q[1];
  }
}

template <bool VEC>
__device__ __forceinline__ void prologue8(const void* x, int x_dtype, size_t xe,
                                          const uint16_t* sp, uint16_t* dst, bool live,
                                          int lane) {
  if constexpr (VEC) {
    // f16 activations: packed f16 products (scale8_f16)
    if (x_dtype == DT_F16) {
      float v[8];
      scale8_f16(*(const u32x4*)((const uint16_t*)x + xe), *(const u32x4*)sp, v);
      finish8_scaled<VEC>(v, dst, live, lane);
      return;
    }
  }
  float a[8], sv[8];
  load8<VEC>(x, x_dtype, xe, sp, a, sv);
  finish8<VEC>(a, sv, dst, live, lane);
}

// prologue8 split into its loads and its arithmetic, for 16-byte aligned x and
// scales: the loads of a lane's 8 activations (one 16-byte load, two for f32)
// and 8 scales are issued early and consumed by pro8_finish, which stores the
// lane's 8 xhat values as one 16-byte write when `live`.  The results equal
// prologue8's.  All 16 lanes of the DPP row must be active.
struct Pro8In {
  u32x4 x0, x1, s;  // x1: the high 16 bytes of f32 activations
};
__device__ __forceinline__ Pro8In pro8_load(const void* x, int x_dtype, size_t xe,
                                            const uint16_t* sp) {
  Pro8In in;
  if (x_dtype == DT_F32) {
    const u32x4* xp = (const u32x4*)((const float*)x + xe);
    in.x0 = xp[0];
    in.x1 = xp[1];
  } else {
    in.x0 = *(const u32x4*)((const uint16_t*)x + xe);
    in.x1 = in.x0;
  }
  in.s = *(const u32x4*)sp;
  return in;
}
__device__ __forceinline__ void pro8_finish(const Pro8In& in, int x_dtype, uint16_t* dst,
                                            bool live, int lane) {
  float v[8];
  if (x_dtype == DT_F16) {
    scale8_f16(in.x0, in.s, v);
  } else {
    float sv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t si = in.s[i];
      sv[2 * i] = h2f((uint16_t)si);
      sv[2 * i + 1] = h2f((uint16_t)(si >> 16));
    }
    if (x_dtype == DT_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = in.x0[i], hi = in.x1[i];
        v[i] = round_f16(round_f16(__builtin_bit_cast(float, lo)) * sv[i]);
        v[i + 4] = round_f16(round_f16(__builtin_bit_cast(float, hi)) * sv[i + 4]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t xi = in.x0[i];
        v[2 * i] = round_f16(round_f16(bf2f((uint16_t)xi)) * sv[2 * i]);
        v[2 * i + 1] = round_f16(round_f16(bf2f((uint16_t)(xi >> 16))) * sv[2 * i + 1]);
      }
    }
  }
  finish8_scaled<true>(v, dst, live, lane);
}

#ifdef EXL3_QMV_PHASES
// Lane 0 of each wave writes its stamps (words 0..6; word 7, the end of the
// epilogue, follows for last arrivers).
__device__ __forceinline__ void phase_record(unsigned long long (&ph)[kPhaseWords], int last,
                                             int lane, int wave, int kw) {
  ph[3] = __builtin_amdgcn_s_memrealtime();
  // HW_ID (wave, SIMD, CU, SH, SE) and XCC_ID, read with s_getreg_b32
  const unsigned long long hw = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);
  const unsigned long long xcc = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xffu;
  ph[6] = hw | xcc << 32 | (unsigned long long)(last != 0) << 48;
  if (qmv_phase_out && lane == 0) {
    unsigned long long* o =
        qmv_phase_out + ((size_t)(blockIdx.y * gridDim.x + blockIdx.x) * 4 * kw + wave) * kPhaseWords;
#pragma unroll
    for (int i = 0; i < 7; ++i) o[i] = ph[i];
  }
}
#endif

// KW waves share each column pair and split the workgroup's K-range between
// them (reduced through LDS in a fixed order), so a workgroup of 4*KW waves
// amortises one prologue over KW times more weight stream.
// MULTI = false is the single-row variant of a plain launch (the batch-1
// decode): no batched prologue or epilogue code, no separate prologue and no
// SwiGLU edge.  FRAG (multi-row only) exchanges the split-K partials in
// fragment order instead of row-major.  SHALLOW (KW = 1; chosen by the host
// from 3 waves per SIMD) keeps one slice per prefetch set: each wave's step
// then takes that much longer, so shallower prefetch still covers the memory
// latency (4096x14336 at 3.5 waves per SIMD: 13.85 -> 13.64 us; at 1 or 1.75
// waves per SIMD it is slower), and decodes its first step before the
// prologue's barrier (PEEL).  The row-major multi-row kernel (MULTI, !FRAG)
// asks for 5 waves per SIMD: left alone its epilogue took it to 104 registers
// and 4 waves, which launches of more than 4 waves per SIMD felt (27648x5120
// M=4, 4320 waves: 36.2 -> 32.5 us; C5 layer M=4 K2/K4 117.1/124.7 ->
// 111.8/116.6 us; 90 registers, no scratch).
template <int K, int CB, int KW, bool MULTI, bool FRAG, bool SHALLOW = false>
__global__ __launch_bounds__(256 * KW)
__attribute__((amdgpu_waves_per_eu(MULTI && !FRAG && KW == 1 ? 5 : 1))) void qmv_kernel(
    QmvParams p) {
  static_assert(MULTI || !FRAG, "the fragment exchange is a multi-row form");
  extern __shared__ __attribute__((aligned(16))) _Float16 xs[];  // [M][rows of split]
  __shared__ int s_last;
  __shared__ float4v red[KW > 1 ? KW - 1 : 1][4][2][64];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pair = wave & 3, kpart = wave >> 2;
  const int cblk = blockIdx.x, split = blockIdx.y;  // global column block
  const Member mm = select_member(p, cblk);
  const int cblk_l = cblk - mm.cblk0;  // column block inside the member
  const int TN = mm.out >> 4, NB = p.in >> 7;
  const int b0 = split * NB / p.splits, b1 = (split + 1) * NB / p.splits;
  const int row0 = b0 * 128, nrows = (b1 - b0) * 128, nq_wg = nrows >> 6;
  // the K-part's quads (one K-part: the workgroup's, a uniform range)
  const int q_lo = KW == 1 ? 0 : kpart * nq_wg / KW;
  const int q_hi = KW == 1 ? nq_wg : (kpart + 1) * nq_wg / KW;
  const int nquads = q_hi - q_lo;
  const int M = p.M;
  EXL3_PHASE(unsigned long long ph[kPhaseWords] = {};
             ph[0] = __builtin_amdgcn_s_memrealtime();)
  // Issue priority falls with progress (3 -> 0 over the K-range): the SIMD's
  // arbiter otherwise favours the oldest wave, which starves later waves until
  // it finishes and leaves them to run alone at single-wave efficiency.
  __builtin_amdgcn_s_setprio(3);

  // The activation loads of the wave's first kPrologueEarly prologue jobs go
  // out first, then the weight stream's first set, so the Hadamards below wait
  // only for the (shared, cache-resident) activations, not behind the weights.
  constexpr int kPrologueEarly = 2;
  const int nb = b1 - b0;
  // Multi-row calls get xhat from a separate prologue launch (mm.xhat): the
  // fused prologue would be repeated by every column block, M times over.
  const bool pre = MULTI && mm.xhat != nullptr;
  const int njobs = pre ? 0 : M * nb;
  PrologueIn first[kPrologueEarly];
  if (!pre) {
#pragma unroll
    for (int t = 0; t < kPrologueEarly; ++t) {
      // a second early job only where the workgroup has one (uniform)
      if (t == 0 || njobs > 4 * KW) {
        const int job = min(wave + t * 4 * KW, njobs - 1);  // clamped: always a valid job
        const int m = job / nb, b = job - m * nb;
        first[t] = prologue_load(p.x, p.x_dtype, (size_t)m * p.in + row0 + b * 128, mm.suh,
                                 row0 + b * 128, lane);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7;
  const size_t qstride = (size_t)4 * TN * 8 * K;  // words per quad of tile rows
  // The weight loads are buffer loads from the workgroup's base (its first
  // tile row and column block: uniform, so the resource sits in scalar
  // registers), bounded by the end of the member's trellis.  A lane's byte
  // offset holds everything that depends on the wave (column pair, K-part) and
  // the lane; a quad's offset is scalar with one K-part and joins the lane's
  // offset otherwise.
  const size_t wg_words = ((size_t)(row0 >> 4) * TN + cblk_l * 8) * (8 * K);
  const size_t tensor_words = (size_t)NB * 8 * TN * (8 * K);
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(mm.trellis + wg_words), 0,
      (int)(uint32_t)min((tensor_words - wg_words) * 4, (size_t)0xffffffffu), kBufferRsrcWord3);
  const uint32_t loff = (uint32_t)((((size_t)4 * q_lo * TN + pair * 2 + g * TN + hsel) * 8 * K +
                                    j * K) * 4);
  const uint32_t loff_prev = loff + (uint32_t)((j == 0 ? 8 * K - 1 : -1) * 4);
  constexpr int D = SHALLOW ? 1 : kQmvLoopDepth<K>;
  uint32_t setA[D][K + 1], setB[D][K + 1];
  const int qlast = nquads > 0 ? nquads - 1 : 0;
  const uint32_t qbytes = (uint32_t)qstride * 4u, last_off = (uint32_t)qlast * qbytes;
  auto fetch_slice = [&](uint32_t(&set)[K + 1], int q) {
    const uint32_t o = min((uint32_t)q * qbytes, last_off);  // past-the-end quads re-read the last
    if constexpr (KW == 1)
      load_slice_prev_b<K>(wrsrc, o, loff, loff_prev, set);
    else
      load_slice_prev_b<K>(wrsrc, 0, loff + o, loff_prev + o, set);
  };
  // SHALLOW launches (3+ waves per SIMD): the first set's B fragments are decoded
  // before the barrier that publishes xhat (the decode needs no activations),
  // with the second set's loads already out: issued here, before the
  // prologue's Hadamards, where K's states need a window each (16 % K != 0:
  // one load per word and a costlier decode), after them otherwise.  Same-box
  // A/B at 4096x14336 M=1 (us), before -> after them / here: K=2 13.22 ->
  // 13.03 / 13.06, K=3 15.26 -> 15.18 / 14.69, K=4 13.35 -> 13.06 / 13.28,
  // K=5 24.30 -> 24.28 / 23.28, K=6 26.83 -> 26.82 / 25.50, K=8 22.03 ->
  // 22.02 / 22.13; bit-identical.  With D = 2 (one wave per SIMD, 4096x4096)
  // the early decode cost 2 % (8.44 -> 8.61 us), so it stays off there.
  constexpr bool PEEL = SHALLOW;
  constexpr bool kEarlySecond = PEEL && 16 % K != 0;
#pragma unroll
  for (int d = 0; d < D; ++d) fetch_slice(setA[d], d);
  if constexpr (kEarlySecond) {
#pragma unroll
    for (int d = 0; d < D; ++d) fetch_slice(setB[d], D + d);
  }
  __builtin_amdgcn_sched_barrier(0);

  // prologue into LDS
  if (pre) {
    const int chunks = nrows >> 3, total = M * chunks;  // 16-byte chunks per row
    if constexpr (FRAG) {
      // 8+ rows: kCopyBatch of a thread's chunks in flight together, as buffer
      // loads (the compiler re-rolls plain ones into one load per iteration),
      // clamped to a valid chunk and stored only where real.  Not in the
      // row-major kernels: the same code there cost 4 % at M = 4 (5120x5120
      // 13.16 -> 13.72 us) although that path never runs at those rows.
      constexpr int kCopyBatch = 4;
      const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(mm.xhat + row0), 0, (int)min((size_t)M * p.in * 2, (size_t)0x7fffffff),
          kBufferRsrcWord3);
      for (int i0 = threadIdx.x; i0 < total; i0 += kCopyBatch * 256 * KW) {
        u32x4 v[kCopyBatch];
#pragma unroll
        for (int u = 0; u < kCopyBatch; ++u) {
          const int i = min(i0 + u * 256 * KW, total - 1);
          const int m = i / chunks, c = i - m * chunks;
          v[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)(m * p.in + c * 8) * 2u, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < kCopyBatch; ++u) {
          const int i = i0 + u * 256 * KW;
          if (i < total) {
            const int m = i / chunks, c = i - m * chunks;
            *(u32x4*)(xs + m * nrows + c * 8) = v[u];
          }
        }
      }
    } else {
      for (int i = threadIdx.x; i < total; i += 256 * KW) {
        const int m = i / chunks, c = i - m * chunks;
        *(u32x4*)(xs + m * nrows + c * 8) =
            *(const u32x4*)(mm.xhat + (size_t)m * p.in + row0 + c * 8);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kPrologueEarly; ++t) {
    const int job = wave + t * 4 * KW;
    if (job < njobs) {
      const int m = job / nb, b = job - m * nb;
      float v0, v1;
      prologue_finish(first[t], p.x_dtype, lane, v0, v1);
      xs[m * nrows + b * 128 + lane] = (_Float16)v0;
      xs[m * nrows + b * 128 + lane + 64] = (_Float16)v1;
    }
  }
  if constexpr (MULTI) {
    // the remaining jobs (multi-row calls) in batches whose loads are in
    // flight together
    constexpr int kPrologueBatch = 4;
    for (int j0 = wave + kPrologueEarly * 4 * KW; j0 < njobs; j0 += kPrologueBatch * 4 * KW) {
      PrologueIn in[kPrologueBatch];
#pragma unroll
      for (int t = 0; t < kPrologueBatch; ++t) {
        const int job = min(j0 + t * 4 * KW, njobs - 1);  // clamped: always a valid job
        const int m = job / nb, b = job - m * nb;
        in[t] = prologue_load(p.x, p.x_dtype, (size_t)m * p.in + row0 + b * 128, mm.suh,
                              row0 + b * 128, lane);
      }
#pragma unroll
      for (int t = 0; t < kPrologueBatch; ++t) {
        const int job = j0 + t * 4 * KW;
        if (job < njobs) {
          const int m = job / nb, b = job - m * nb;
          float v0, v1;
          prologue_finish(in[t], p.x_dtype, lane, v0, v1);
          xs[m * nrows + b * 128 + lane] = (_Float16)v0;
          xs[m * nrows + b * 128 + lane + 64] = (_Float16)v1;
        }
      }
    }
  } else {
    for (int job = wave + kPrologueEarly * 4 * KW; job < njobs; job += 4 * KW) {
      const int m = job / nb, b = job - m * nb;
      const PrologueIn in = prologue_load(p.x, p.x_dtype, (size_t)m * p.in + row0 + b * 128,
                                          mm.suh, row0 + b * 128, lane);
      float v0, v1;
      prologue_finish(in, p.x_dtype, lane, v0, v1);
      xs[m * nrows + b * 128 + lane] = (_Float16)v0;
      xs[m * nrows + b * 128 + lane + 64] = (_Float16)v1;
    }
  }
  half8 first_b[PEEL ? D : 1][4];  // the first set's fragments (PEEL)
  if constexpr (PEEL) {
    if constexpr (!kEarlySecond) {
#pragma unroll
      for (int d = 0; d < D; ++d) fetch_slice(setB[d], D + d);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) decode_step<K, CB>(setA[d], first_b[d]);
  }
  __syncthreads();
  EXL3_PHASE(ph[1] = __builtin_amdgcn_s_memrealtime(); ph[4] = __builtin_amdgcn_s_memtime();)

  // main loop: two sets of D slices in ping-pong; the D loads of one set are
  // issued together, then the other set (already in flight for D steps) is
  // decoded, so a wait at any point still has D steps of decode behind it.
  // A rows >= M read row M-1: MFMA output rows depend only on their own A
  // row, and rows >= M are never stored.
  const int am = min(lane & 15, M - 1);
  const _Float16* xrow = xs + (size_t)am * nrows + 64 * q_lo + g * 16;
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  // issue priority falls at the quarters of the K-range (steps t1, t2, t3),
  // set after each set of D steps, when the launch puts more than one wave on
  // a SIMD (p.prio_ramp): a lone wave gains nothing from it and loses the
  // setprio issue slots (4096x4096, one wave per SIMD: 8.54 -> 8.17 us without)
  const int t1 = (nquads + 3) / 4, t2 = (2 * nquads + 3) / 4, t3 = (3 * nquads + 3) / 4;
  auto lower_priority = [&](int done) {
    if (done >= t3) __builtin_amdgcn_s_setprio(0);
    else if (done >= t2) __builtin_amdgcn_s_setprio(1);
    else if (done >= t1) __builtin_amdgcn_s_setprio(2);
  };
  // A whole set is one branch-free block, so the compiler interleaves the
  // decode chains of its D steps; only the last, partial pass tests each step.
  auto compute = [&](uint32_t(&set)[D][K + 1], int qbase, bool whole) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int q = qbase + d;
      if (whole || q < nquads) {
        half8 a0 = *(const half8*)(xrow + q * 64);
        half8 a1 = *(const half8*)(xrow + q * 64 + 8);
        qmv_step_prev<K, CB>(set[d], a0, a1, acc0, acc1);
      }
    }
    if (p.prio_ramp) lower_priority(qbase + D);
  };
  // Unconditional loads (past-the-end quads re-read the last one) keep the
  // load count static, so the waits before each decode can be partial.
  auto fetch = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d) fetch_slice(set[d], qbase + d);
  };
  int q0 = 0;
  if constexpr (PEEL) {  // the first set was decoded before the barrier; setB is in flight
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < nquads)
        mma_step(*(const half8*)(xrow + d * 64), *(const half8*)(xrow + d * 64 + 8), first_b[d],
                 acc0, acc1);
    if (p.prio_ramp) lower_priority(D);
    fetch(setA, 2 * D);
    compute(setB, D, false);
    q0 = 2 * D;
  }
  for (; q0 + 2 * D <= nquads; q0 += 2 * D) {
    fetch(setB, q0 + D);
    compute(setA, q0, true);
    fetch(setA, q0 + 2 * D);
    compute(setB, q0 + D, true);
  }
  if (q0 < nquads) {  // fewer than 2*D steps left; setA holds step q0's slices
    fetch(setB, q0 + D);
    compute(setA, q0, false);
    compute(setB, q0 + D, false);
  }

  EXL3_PHASE(ph[2] = __builtin_amdgcn_s_memrealtime(); ph[5] = __builtin_amdgcn_s_memtime();)
  // K-parts of a pair meet in LDS; part 0 adds them in part order
  if constexpr (KW > 1) {
    if (kpart > 0) {
      red[kpart - 1][pair][0][lane] = acc0;
      red[kpart - 1][pair][1][lane] = acc1;
    }
    __syncthreads();
#pragma unroll
    for (int kp = 0; kp < KW - 1; ++kp) {
      acc0 += red[kp][pair][0][lane];
      acc1 += red[kp][pair][1][lane];
    }
  }
  // every wave stays to the end (each barrier is reached by the whole
  // workgroup); only K-part 0 stores and finishes
  const bool writer = kpart == 0;

  // accumulator lane l: rows 4*(l/16)+r, column 16*(tn0 + n/8) + n%8 + 8*cg
  // (tn0 = cblk_l*8 + 2*pair, the pair's first tile)
  // of the member; partials are laid out by global column
  const int n = lane & 15;
  const int col = 128 * cblk + 16 * (pair * 2 + (n >> 3)) + (n & 7);
  const int TO = p.total_out;
  // FRAG: partials in fragment order, a slab of 8 KB per (split, column
  // block): [pair][acc0, acc1][lane] of 16 bytes, one coalesced coherent
  // 16-byte store per accumulator.  Otherwise row-major, 4 bytes per value.
  auto frag_slab = [&](int sp, int gcb) {
    return __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.partials + ((size_t)sp * (TO >> 7) + gcb) * 2048), 0, 8192, kBufferRsrcWord3);
  };
  if constexpr (FRAG) {
    if (writer) {
      const __amdgpu_buffer_rsrc_t mine = frag_slab(split, cblk);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc0), mine,
                                             ((pair * 2) * 64 + lane) * 16, 0, kCpolSc1);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc1), mine,
                                             ((pair * 2 + 1) * 64 + lane) * 16, 0, kCpolSc1);
    }
  } else {
    float* part = p.partials + (size_t)split * M * TO;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int m = 4 * g + r;
      if (writer && m < M) {
        store_coherent(part + (size_t)m * TO + col, acc0[r]);
        store_coherent(part + (size_t)m * TO + col + 8, acc1[r]);
      }
    }
  }

  // last workgroup of this column block finishes it.  Partials and counters
  // are exchanged only through agent-scope coherent accesses (sc1 loads and
  // stores, relaxed atomics: served at the device coherence point, no L2
  // writeback); s_waitcnt + barrier order every
  // partial store of the workgroup before its counter increment.
  // A SwiGLU group finishes a column block once both members' splits are in
  // (one counter per block pair).
  const bool glu = MULTI && p.glu.on;
  const int arrivals = glu ? 2 * p.splits : p.splits;
  const int cidx = glu ? cblk_l : cblk;
  if (arrivals > 1) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t old = __hip_atomic_fetch_add(&p.counters[cidx], 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (uint32_t)(arrivals - 1));
    }
    __syncthreads();
#ifdef EXL3_QMV_PHASES
    if (!MULTI) phase_record(ph, s_last, lane, wave, KW);
#endif
    if (!s_last) return;  // uniform across the workgroup
    if (threadIdx.x == 0)
      __hip_atomic_store(&p.counters[cidx], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#ifdef EXL3_QMV_PHASES
    if (!MULTI) phase_record(ph, 1, lane, wave, KW);
#endif
  }
  const int colb_l = cblk_l * 128;
  // Split sums: the loads of kSplitChunk splits go out together (one round
  // trip to the coherence point per chunk, not per split); the adds stay in
  // split order.
  auto sum_row = [&](int m, int colg, float& v0, float& v1) {
    v0 = 0.f;
    v1 = 0.f;
    sum_split_columns(p.partials + (size_t)m * TO + colg, (size_t)M * TO, p.splits, lane, v0, v1);
  };
  // a (gate, up) row of the block: staged H128, *svh, +bias, f16 SwiGLU and,
  // for the fused MLP, the down projection's prologue
  auto glu_finish = [&](int m, float g0, float g1, float u0, float u1) {
    const Member& gm = p.mem[0];
    const Member& um = p.mem[1];
    const int H = gm.out;
    finish_vals128(g0, g1, lane, colb_l, gm.svh);
    finish_vals128(u0, u1, lane, colb_l, um.svh);
    g0 = with_bias_f16(g0, gm.bias, colb_l + lane);
    g1 = with_bias_f16(g1, gm.bias, colb_l + lane + 64);
    u0 = with_bias_f16(u0, um.bias, colb_l + lane);
    u1 = with_bias_f16(u1, um.bias, colb_l + lane + 64);
    float a0 = swiglu_f16(g0, u0), a1 = swiglu_f16(g1, u1);
    if (p.glu.down_suh) {  // the down projection's prologue on this 128-block
      a0 = round_f16(a0 * h2f(p.glu.down_suh[colb_l + lane]));
      a1 = round_f16(a1 * h2f(p.glu.down_suh[colb_l + lane + 64]));
      h128_wave<true>(a0, a1, lane);
      a0 = round_f16(a0 * kHadScale);
      a1 = round_f16(a1 * kHadScale);
    }
    p.glu.out[(size_t)m * H + colb_l + lane] = f2h(a0);
    p.glu.out[(size_t)m * H + colb_l + lane + 64] = f2h(a1);
  };
  if constexpr (!MULTI) {  // the plain single-row epilogue (no SwiGLU edge)
    for (int m = wave; m < M; m += 4 * KW) {
      float v0, v1;
      sum_row(m, cblk * 128, v0, v1);
      finish_row128(v0, v1, lane, colb_l, mm.svh, mm.bias, mm.y, mm.y_dtype, p.x_dtype,
                    (size_t)m * mm.out);
    }
#ifdef EXL3_QMV_PHASES
    __builtin_amdgcn_s_waitcnt(0);  // the output stores have landed
    if (qmv_phase_out && lane == 0)
      qmv_phase_out[((size_t)(blockIdx.y * gridDim.x + blockIdx.x) * 4 * KW + wave) * kPhaseWords +
                    7] = __builtin_amdgcn_s_memrealtime();
#endif
  } else if constexpr (!FRAG) {
    // rows of the block from row-major partials (the split loads of a batch go
    // out together, each row adding its splits in split order)
    if (!p.glu.on) {
      // rows in batches of 4 per wave: the split sums of a batch load together,
      // kRowChunk splits at a time (each row still adds its splits in split
      // order)
      constexpr int kRows = 4, kRowChunk = kSplitChunk / 2;
      for (int m0 = wave; m0 < M; m0 += kRows * 4 * KW) {
        float v0[kRows], v1[kRows];
#pragma unroll
        for (int t = 0; t < kRows; ++t) v0[t] = v1[t] = 0.f;
        for (int s0 = 0; s0 < p.splits; s0 += kRowChunk) {
          float a[kRowChunk][kRows], b[kRowChunk][kRows];
#pragma unroll
          for (int i = 0; i < kRowChunk; ++i) {
            const int sp = min(s0 + i, p.splits - 1);  // clamped: always a written split
#pragma unroll
            for (int t = 0; t < kRows; ++t) {
              const int m = min(m0 + t * 4 * KW, M - 1);  // clamped: always a written row
              const float* ps = p.partials + ((size_t)sp * M + m) * TO + cblk * 128;
              a[i][t] = load_coherent(ps + lane);
              b[i][t] = load_coherent(ps + lane + 64);
            }
          }
#pragma unroll
          for (int i = 0; i < kRowChunk; ++i)
            if (s0 + i < p.splits)
#pragma unroll
              for (int t = 0; t < kRows; ++t) {
                v0[t] += a[i][t];
                v1[t] += b[i][t];
              }
        }
#pragma unroll
        for (int t = 0; t < kRows; ++t) {
          const int m = m0 + t * 4 * KW;
          if (m < M)
            finish_row128(v0[t], v1[t], lane, colb_l, mm.svh, mm.bias, mm.y, mm.y_dtype,
                          p.x_dtype, (size_t)m * mm.out);
        }
      }
      return;
    }
    for (int m = wave; m < M; m += 4 * KW) {
      float g0, g1, u0, u1;
      sum_row(m, (p.mem[0].cblk0 + cblk_l) * 128, g0, g1);
      sum_row(m, (p.mem[1].cblk0 + cblk_l) * 128, u0, u1);
      glu_finish(m, g0, g1, u0, u1);
    }
  } else {
    // Multi-row: the split sums in fragment space -- pair wave w (K-part 0)
    // loads its two accumulators of every split (16-byte coherent loads, up to
    // kSplitChunk / 2 splits in flight) and adds them in split order -- then the
    // block's rows through LDS to the row-wise finishing.  The rows (M per
    // member, f32) take the activation buffer's place: every wave is past
    // the K loop (the barrier above).
    float(*const ysum)[128] = reinterpret_cast<float(*)[128]>(xs);
    auto gather_block = [&](int gcb, float(*dst)[128]) {
      if (writer) {
        float4v s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
        // kFragChunk splits' two fragments in flight (16 bytes each: 8 splits
        // would hold 64 more registers and cost the kernel a wave per SIMD)
        constexpr int kFragChunk = kSplitChunk / 2;
        for (int c0 = 0; c0 < p.splits; c0 += kFragChunk) {
          float4v a[kFragChunk], b[kFragChunk];
#pragma unroll
          for (int i = 0; i < kFragChunk; ++i) {
            const __amdgpu_buffer_rsrc_t src = frag_slab(min(c0 + i, p.splits - 1), gcb);
            a[i] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                   src, ((pair * 2) * 64 + lane) * 16, 0, kCpolSc1));
            b[i] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                   src, ((pair * 2 + 1) * 64 + lane) * 16, 0,
                                                   kCpolSc1));
          }
#pragma unroll
          for (int i = 0; i < kFragChunk; ++i) {
            s0 = add_if(c0 + i < p.splits, s0, a[i]);
            s1 = add_if(c0 + i < p.splits, s1, b[i]);
          }
        }
        const int c = 16 * (pair * 2 + (n >> 3)) + (n & 7);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * g + r < M) {
            dst[4 * g + r][c] = s0[r];
            dst[4 * g + r][c + 8] = s1[r];
          }
      }
    };
    if (!p.glu.on) {
      gather_block(cblk, ysum);
      __syncthreads();
      for (int m = wave; m < M; m += 4 * KW)
        finish_row128(ysum[m][lane], ysum[m][lane + 64], lane, colb_l, mm.svh, mm.bias, mm.y,
                      mm.y_dtype, p.x_dtype, (size_t)m * mm.out);
      return;
    }
    float(*const usum)[128] = ysum + M;
    gather_block(p.mem[0].cblk0 + cblk_l, ysum);
    gather_block(p.mem[1].cblk0 + cblk_l, usum);
    __syncthreads();
    for (int m = wave; m < M; m += 4 * KW)
      glu_finish(m, ysum[m][lane], ysum[m][lane + 64], usum[m][lane], usum[m][lane + 64]);
  }
}

// Decode hook (the reference's `metal-decode` codec op, exl3.metal:102-109):
// states and f16 values of every tile in tile order, computed with the exact
// per-lane window/decode code the QMV and QMM kernels use.  8 lanes per tile.
template <int K, int CB>
__global__ __launch_bounds__(256) void decode_tiles_kernel(const uint32_t* __restrict__ packed,
                                                           int64_t tiles,
                                                           uint16_t* __restrict__ states,
                                                           uint16_t* __restrict__ values) {
  const int lane = threadIdx.x & 63;
  const int64_t slot = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;  // tile
  const int j = threadIdx.x & 7;
  const bool live = slot < tiles;
  uint32_t w[K];
#pragma unroll
  for (int i = 0; i < K; ++i) w[i] = live ? packed[slot * 8 * K + j * K + i] : 0u;
  uint32_t B[K + 1];
  B[0] = prev_word(w[K - 1], lane);  // every lane takes part in the permute
#pragma unroll
  for (int i = 0; i < K; ++i) B[i + 1] = w[i];
  if (!live) return;
  uint32_t src[32];
  extract_states<K>(B, src);
  const int64_t base = slot * 256 + j * 32;
  if (states) {
    static_for<32>([&](auto S_) {
      constexpr int S = decltype(S_)::value;
      states[base + S] = (uint16_t)state_value<K, S>(src);
    });
  }
  static_for<16>([&](auto P_) {
    constexpr int P = decltype(P_)::value;
    uint32_t d = decode_pair<CB, K, 2 * P>(src);
    *(uint32_t*)(values + base + 2 * P) = d;
  });
}

// Codewords of arbitrary 16-bit states (the reference's `codebook` codec op,
// codec.rs:52-71), with the decode code the kernels use (state in the low
// half of a window).
template <int CB>
__global__ __launch_bounds__(256) void codewords_kernel(const uint16_t* __restrict__ states,
                                                        int64_t n, uint16_t* __restrict__ values) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t src[32];
  src[0] = states[i];
  values[i] = (uint16_t)decode_one<CB, 3, 0>(src);  // K = 3: state 0 sits in the low half
}

}  // namespace exl3
