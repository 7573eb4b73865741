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
//      them with up to 16 activation rows at once (rows >= M are zero), so
//      M = 1..16 costs the same decode;
//   3. split-K partials go to the workspace; the last workgroup to finish a
//      128-column block sums the splits in split order (deterministic), and
//      applies the epilogue (linear.rs:984-997): f16, H128, * svh, cast, bias.
#pragma once

#include "exl3_device.hpp"
#include "exl3_params.hpp"

namespace exl3 {


// Load the K words of this lane's slice of a tile.
template <int K>
__device__ __forceinline__ void load_slice(const uint32_t* __restrict__ p, uint32_t (&w)[K]) {
  if constexpr (K == 4) {
    u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
  } else if constexpr (K == 8) {
    u32x4 v0 = __builtin_nontemporal_load((const u32x4*)p);
    u32x4 v1 = __builtin_nontemporal_load((const u32x4*)p + 1);
    w[0] = v0[0], w[1] = v0[1], w[2] = v0[2], w[3] = v0[3];
    w[4] = v1[0], w[5] = v1[1], w[6] = v1[2], w[7] = v1[3];
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) w[i] = __builtin_nontemporal_load(p + i);
  }
}

// Decode the 4 B fragments of one 8-tile load and run the 4 MFMAs.
template <int K, int CB>
__device__ __forceinline__ void qmv_step(const uint32_t (&w)[K], int lane, half8 a0, half8 a1,
                                         float4v& acc0, float4v& acc1) {
  uint32_t B[K + 1];
  B[0] = prev_word(w[K - 1], lane);
#pragma unroll
  for (int i = 0; i < K; ++i) B[i + 1] = w[i];
  uint32_t src[32];
  extract_states<K>(B, src);
  half8 b00 = decode_fragment<CB, K, 0, 0>(src);
  half8 b01 = decode_fragment<CB, K, 0, 1>(src);
  acc0 = mfma16(a0, b00, acc0);
  acc1 = mfma16(a0, b01, acc1);
  half8 b10 = decode_fragment<CB, K, 1, 0>(src);
  half8 b11 = decode_fragment<CB, K, 1, 1>(src);
  acc0 = mfma16(a1, b10, acc0);
  acc1 = mfma16(a1, b11, acc1);
}

// Epilogue for one row of a 128-column block held as (v0, v1) = columns
// (lane, lane+64): f16(sum) -> staged H128 -> f16(*1/sqrt128) -> f16(*svh)
// -> cast (+bias).
__device__ __forceinline__ void finish_row128(float v0, float v1, int lane, int col0,
                                              const uint16_t* __restrict__ svh,
                                              const uint16_t* __restrict__ bias, void* y,
                                              int y_dtype, size_t row_off) {
  v0 = round_f16(v0);
  v1 = round_f16(v1);
  h128_wave<true>(v0, v1, lane);
  v0 = round_f16(v0 * kHadScale);
  v1 = round_f16(v1 * kHadScale);
  int c0 = col0 + lane, c1 = col0 + lane + 64;
  v0 = round_f16(v0 * h2f(svh[c0]));
  v1 = round_f16(v1 * h2f(svh[c1]));
  store_out(y, y_dtype, row_off + c0, v0, bias, c0);
  store_out(y, y_dtype, row_off + c1, v1, bias, c1);
}

// Prologue for one row of one 128-input block: returns xhat for elements
// (lane, lane+64) of the block.
__device__ __forceinline__ void prepare_row128(const void* x, int x_dtype, size_t off,
                                               const uint16_t* __restrict__ suh, int e0, int lane,
                                               float& v0, float& v1) {
  v0 = round_f16(round_f16(load_act(x, x_dtype, off + lane)) * h2f(suh[e0 + lane]));
  v1 = round_f16(round_f16(load_act(x, x_dtype, off + lane + 64)) * h2f(suh[e0 + lane + 64]));
  h128_wave<true>(v0, v1, lane);
  v0 = round_f16(v0 * kHadScale);
  v1 = round_f16(v1 * kHadScale);
}

template <int K, int CB>
__global__ __launch_bounds__(256) void qmv_kernel(QmvParams p) {
  extern __shared__ __attribute__((aligned(16))) _Float16 xs[];  // [M][rows of split]
  __shared__ int s_last;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int TN = p.out >> 4, NB = p.in >> 7;
  const int cblk = blockIdx.x, split = blockIdx.y;
  const int b0 = split * NB / p.splits, b1 = (split + 1) * NB / p.splits;
  const int row0 = b0 * 128, nrows = (b1 - b0) * 128, nquads = nrows >> 6;
  const int M = p.M;

  // weight stream pointers; first loads go out before the prologue
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7;
  const int tn0 = cblk * 8 + wave * 2;
  const size_t qstride = (size_t)4 * TN * 8 * K;
  const uint32_t* tp =
      p.trellis + ((size_t)((row0 >> 4) + g) * TN + tn0 + hsel) * (8 * K) + (size_t)j * K;
  uint32_t wa[K], wb[K];
  load_slice<K>(tp, wa);
  if (nquads > 1) load_slice<K>(tp + qstride, wb);

  // prologue into LDS
  const int nb = b1 - b0;
  for (int job = wave; job < M * nb; job += 4) {
    int m = job / nb, b = job - m * nb;
    float v0, v1;
    prepare_row128(p.x, p.x_dtype, (size_t)m * p.in + row0 + b * 128, p.suh, row0 + b * 128, lane,
                   v0, v1);
    xs[m * nrows + b * 128 + lane] = (_Float16)v0;
    xs[m * nrows + b * 128 + lane + 64] = (_Float16)v1;
  }
  __syncthreads();

  // main loop
  const int am = lane & 15;
  const bool arow = am < M;
  const _Float16* xrow = xs + (size_t)am * nrows + g * 16;
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const half8 zero8 = {};
  for (int q = 0; q < nquads; q += 2) {
    {
      half8 a0 = arow ? *(const half8*)(xrow + q * 64) : zero8;
      half8 a1 = arow ? *(const half8*)(xrow + q * 64 + 8) : zero8;
      uint32_t cur[K];
#pragma unroll
      for (int i = 0; i < K; ++i) cur[i] = wa[i];
      if (q + 2 < nquads) load_slice<K>(tp + (size_t)(q + 2) * qstride, wa);
      qmv_step<K, CB>(cur, lane, a0, a1, acc0, acc1);
    }
    if (q + 1 < nquads) {
      half8 a0 = arow ? *(const half8*)(xrow + (q + 1) * 64) : zero8;
      half8 a1 = arow ? *(const half8*)(xrow + (q + 1) * 64 + 8) : zero8;
      uint32_t cur[K];
#pragma unroll
      for (int i = 0; i < K; ++i) cur[i] = wb[i];
      if (q + 3 < nquads) load_slice<K>(tp + (size_t)(q + 3) * qstride, wb);
      qmv_step<K, CB>(cur, lane, a0, a1, acc0, acc1);
    }
  }

  // accumulator lane l: rows 4*(l/16)+r, column 16*(tn0 + n/8) + n%8 + 8*cg
  const int n = lane & 15;
  const int col = 16 * (tn0 + (n >> 3)) + (n & 7);
  float* part = p.partials + (size_t)split * M * p.out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    int m = 4 * g + r;
    if (m < M) {
      part[(size_t)m * p.out + col] = acc0[r];
      part[(size_t)m * p.out + col + 8] = acc1[r];
    }
  }

  // last workgroup of this column block finishes it
  if (p.splits > 1) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      __threadfence();
      uint32_t old = __hip_atomic_fetch_add(&p.counters[cblk], 1u, __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (uint32_t)(p.splits - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (threadIdx.x == 0) p.counters[cblk] = 0u;
  } else {
    __threadfence_block();
    __syncthreads();
  }
  const int colb = cblk * 128;
  for (int m = wave; m < M; m += 4) {
    float v0 = 0.f, v1 = 0.f;
    for (int s = 0; s < p.splits; ++s) {
      const float* ps = p.partials + ((size_t)s * M + m) * p.out + colb;
      v0 += __builtin_nontemporal_load(ps + lane);
      v1 += __builtin_nontemporal_load(ps + lane + 64);
    }
    finish_row128(v0, v1, lane, colb, p.svh, p.bias, p.y, p.y_dtype, (size_t)m * p.out);
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

}  // namespace exl3
