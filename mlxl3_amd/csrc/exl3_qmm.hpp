// Kernels for the EXL3 linear at M > 16 rows (prefill and large verify):
// the reference's QMM family (qmm_tensor, linear.rs:1874-2083, and the
// _qmm_tensor*_kernel.metal variants), re-designed for gfx950.
//
// Workgroup tile: 128 output columns (8 tiles) x 64*MBW rows, full K.
// Per step of 64 input rows (4 tile rows) each of the 4 waves decodes 8 tiles
// (its 2 output tiles x 4 tile rows) into MFMA B fragments and stores them in
// LDS in fragment order (one ds_write_b128 per fragment, conflict-free); after
// one barrier every wave reads all 16 fragments of the step and multiplies them
// with its own 16*MBW activation rows, whose A fragments come straight from the
// f16 xhat rows in global memory.  Each weight is decoded once per workgroup
// and used for 64*MBW rows.  Two LDS buffers let one barrier per step order
// the writes of step q+2 after every read of step q.
//
// The accumulators of a wave hold whole 128-column blocks of its rows, so the
// output epilogue (f16 -> H128 -> * svh -> cast, linear.rs:1940-1963) runs in
// registers: column c of the block sits at lane bits (c & 7) and bit 4 of c,
// register index (c >> 3) & 1 and c >> 5, and the Hadamard stages become
// lane swizzles for strides 1, 2, 4, 16 and register pairs for 8, 32, 64.
#pragma once

#include "exl3_device.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {


// xhat = prologue(x) for all rows: grid (in/128, M), one wave per block row.
__global__ __launch_bounds__(64) void prologue_kernel(const void* __restrict__ x, int x_dtype,
                                                      const uint16_t* __restrict__ suh, int in,
                                                      uint16_t* __restrict__ xhat) {
  const int lane = threadIdx.x;
  const int b = blockIdx.x, m = blockIdx.y;
  float v0, v1;
  prepare_row128(x, x_dtype, (size_t)m * in + b * 128, suh, b * 128, lane, v0, v1);
  xhat[(size_t)m * in + b * 128 + lane] = f2h(v0);
  xhat[(size_t)m * in + b * 128 + lane + 64] = f2h(v1);
}

template <int STRIDE>
__device__ __forceinline__ float bfly_lane(float v, int lane) {
  float p = __shfl_xor(v, STRIDE, 64);
  return (lane & STRIDE) ? p - v : v + p;
}

template <int K, int CB, int MBW>
__global__ __launch_bounds__(256) void qmm_kernel(QmmParams p) {
  __shared__ u32x4 bsh[2][4][4][64];  // [buffer][wave][fragment h*2+cg][lane]

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int TN = p.out >> 4, nquads = p.in >> 6;
  const int cblk = blockIdx.x % p.col_blocks, mtile = blockIdx.x / p.col_blocks;
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7, n = lane & 15;
  const int tn0 = cblk * 8 + wave * 2;
  const size_t qstride = (size_t)4 * TN * 8 * K;
  const uint32_t* tp = p.trellis + ((size_t)g * TN + tn0 + hsel) * (8 * K) + (size_t)j * K;

  const int row_base = mtile * 64 * MBW + wave * 16 * MBW;
  const uint16_t* arow[MBW];
  bool avalid[MBW];
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb) {
    int row = row_base + 16 * mb + n;
    avalid[mb] = row < p.M;
    arow[mb] = p.xhat + (size_t)(avalid[mb] ? row : 0) * p.in + g * 16;  // clamped, in bounds
  }

  float4v acc[MBW][8];
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
    for (int f = 0; f < 8; ++f) acc[mb][f] = float4v{0.f, 0.f, 0.f, 0.f};

  // Software pipeline per step q: the trellis slice of q+2 and the A
  // fragments of q+1 are in flight while step q decodes and multiplies.  All
  // loads are unconditional (clamped to the last step) so waits stay partial.
  uint32_t w0[K], w1[K];
  load_slice<K>(tp, w0);
  load_slice<K>(tp + (size_t)min(1, nquads - 1) * qstride, w1);
  const half8 zero8 = {};
  half8 an[MBW][2];
  auto load_a = [&](int q) {
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) {
      const half8* src = (const half8*)(arow[mb] + min(q, nquads - 1) * 64);
      an[mb][0] = src[0];
      an[mb][1] = src[1];
    }
  };
  load_a(0);
  auto step = [&](uint32_t(&w)[K], int q) {
    const int buf = q & 1;
    half8 a[MBW][2];
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) {
      a[mb][0] = avalid[mb] ? an[mb][0] : zero8;
      a[mb][1] = avalid[mb] ? an[mb][1] : zero8;
    }
    load_a(q + 1);
    {
      uint32_t B[K + 1];
      B[0] = prev_word(w[K - 1], lane);
#pragma unroll
      for (int i = 0; i < K; ++i) B[i + 1] = w[i];
      uint32_t src[32];
      extract_states<K>(B, src);
      load_slice<K>(tp + (size_t)min(q + 2, nquads - 1) * qstride, w);
      bsh[buf][wave][0][lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 0, 0>(src));
      bsh[buf][wave][1][lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 0, 1>(src));
      bsh[buf][wave][2][lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 1, 0>(src));
      bsh[buf][wave][3][lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 1, 1>(src));
    }
    __syncthreads();
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int cg = 0; cg < 2; ++cg) {
          half8 b = __builtin_bit_cast(half8, bsh[buf][w2][h * 2 + cg][lane]);
#pragma unroll
          for (int mb = 0; mb < MBW; ++mb)
            acc[mb][w2 * 2 + cg] = mfma16(a[mb][h], b, acc[mb][w2 * 2 + cg]);
        }
  };
  for (int q = 0; q < nquads; q += 2) {
    step(w0, q);
    if (q + 1 < nquads) step(w1, q + 1);
  }

  // in-register epilogue; v[f] with f = 2*w + cg is column 32w + 16*(n>>3) + 8cg + (n&7)
  const int colb = cblk * 128;
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row_base + 16 * mb + 4 * g + r;
      float v[8];
#pragma unroll
      for (int f = 0; f < 8; ++f) v[f] = round_f16(acc[mb][f][r]);
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        v[f] = bfly_lane<1>(v[f], lane);
        v[f] = bfly_lane<2>(v[f], lane);
        v[f] = bfly_lane<4>(v[f], lane);
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // stride 8: cg pair
        float a0 = v[2 * w], b0 = v[2 * w + 1];
        v[2 * w] = round_f16(a0 + b0);
        v[2 * w + 1] = round_f16(a0 - b0);
      }
#pragma unroll
      for (int f = 0; f < 8; ++f) v[f] = bfly_lane<8>(v[f], lane);  // stride 16
#pragma unroll
      for (int cg = 0; cg < 2; ++cg) {
#pragma unroll
        for (int wl = 0; wl < 4; wl += 2) {  // stride 32: w bit 0
          float a0 = v[2 * wl + cg], b0 = v[2 * (wl + 1) + cg];
          v[2 * wl + cg] = a0 + b0;
          v[2 * (wl + 1) + cg] = a0 - b0;
        }
#pragma unroll
        for (int wl = 0; wl < 2; ++wl) {  // stride 64: w bit 1
          float a0 = v[2 * wl + cg], b0 = v[2 * (wl + 2) + cg];
          v[2 * wl + cg] = round_f16(a0 + b0);
          v[2 * (wl + 2) + cg] = round_f16(a0 - b0);
        }
      }
      if (row < p.M) {
#pragma unroll
        for (int f = 0; f < 8; ++f) {
          const int c = colb + 32 * (f >> 1) + 16 * (n >> 3) + 8 * (f & 1) + (n & 7);
          float o = round_f16(round_f16(v[f] * kHadScale) * h2f(p.svh[c]));
          store_out(p.y, p.y_dtype, (size_t)row * p.out + c, o, p.bias, c);
        }
      }
    }
}

}  // namespace exl3
