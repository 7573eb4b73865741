// Kernels for the EXL3 linear at M > 16 rows (prefill and large verify):
// the reference's QMM family (qmm_tensor, linear.rs:1874-2083, and the
// _qmm_tensor*_kernel.metal variants), re-designed for gfx950.
//
// Workgroup: 8 waves on a tile of 128 output columns (8 tiles) x 64*MB rows
// over one K-range.  Waves 0-3 are producers, waves 4-7 consumers, so each
// SIMD holds one of each and the trellis decode (VALU) of one overlaps the
// MFMAs of the other:
//  * producer w decodes, per step of 64 input rows (4 tile rows), the 8 tiles
//    of output tiles 2w, 2w+1 into MFMA B fragments and stores them in LDS in
//    fragment order (one ds_write_b128 per fragment, conflict-free); its
//    trellis slices are loaded two steps ahead;
//  * consumer w owns 16*MB rows and multiplies them by all 16 fragments of the
//    step, with A fragments read from the f16 xhat rows one step ahead.
// Two LDS buffers and one workgroup barrier per step: producers fill buffer
// (q+1)&1 while consumers read buffer q&1.  Each weight is decoded once per
// 64*MB rows.
//
// The accumulators of a consumer hold whole 128-column blocks of its rows, so
// the output epilogue (f16 -> H128 -> * svh -> cast, linear.rs:1940-1963)
// runs in registers: column c of the block sits at lane bits (c & 7) and bit 4
// of c, register index (c >> 3) & 1 and c >> 5, and the Hadamard stages
// become lane swizzles for strides 1, 2, 4, 16 and register pairs for 8, 32,
// 64.  With a global split-K the K-ranges leave f32 partials (exchanged with
// agent-scope relaxed atomics, as in the QMV) and the last workgroup of an
// output tile adds them in split order, so results do not depend on timing.
#pragma once

#include "exl3_device.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {


// xhat = prologue(x) for all rows.  A job is one (row, 128-input block); a
// wave takes kPrologueJobs jobs spaced by the grid, issues all their loads,
// then runs the Hadamards, so several jobs' memory latencies overlap.
constexpr int kPrologueJobs = 4;
__global__ __launch_bounds__(256) void prologue_kernel(const void* __restrict__ x, int x_dtype,
                                                       const uint16_t* __restrict__ suh, int in,
                                                       int jobs, uint16_t* __restrict__ xhat) {
  const int lane = threadIdx.x & 63;
  const int nb = in >> 7;
  const int stride = gridDim.x * 4;
  const int first = blockIdx.x * 4 + (threadIdx.x >> 6);
  PrologueIn pin[kPrologueJobs];
#pragma unroll
  for (int t = 0; t < kPrologueJobs; ++t) {
    const int job = min(first + t * stride, jobs - 1);  // clamped: loads stay in bounds
    const int m = job / nb, b = job - m * nb;
    pin[t] = prologue_load(x, x_dtype, (size_t)m * in + b * 128, suh, b * 128, lane);
  }
#pragma unroll
  for (int t = 0; t < kPrologueJobs; ++t) {
    const int job = first + t * stride;
    float v0, v1;
    prologue_finish(pin[t], x_dtype, lane, v0, v1);
    if (job < jobs) {
      const int m = job / nb, b = job - m * nb;
      xhat[(size_t)m * in + b * 128 + lane] = f2h(v0);
      xhat[(size_t)m * in + b * 128 + lane + 64] = f2h(v1);
    }
  }
}

template <int STRIDE>
__device__ __forceinline__ float bfly_lane(float v, int lane) {
  float p = xor_lanes<STRIDE>(v);
  return (lane & STRIDE) ? p - v : v + p;
}

// 16-bit output bits of the linear epilogue's final cast (+ bias), as
// store_out computes them.
__device__ __forceinline__ uint32_t out16(float v16, float b, bool has_bias, int dt) {
  if (dt == DT_F16) return f2h(has_bias ? round_f16(v16 + b) : v16);
  float v = bf2f(f2bf(v16));
  if (has_bias) v = v + b;
  return f2bf(v);
}

// One row of a 128-column block: v[f] holds column 32*(f>>1) + 16*(n>>3) +
// 8*(f&1) + (n&7) of the row, n = lane & 15 (f32 sums).  svh and bias of the
// block come from LDS (f32).  All lanes take part in the exchanges; only
// `live` lanes store.  16-bit outputs leave as 32-bit pairs: for each
// register pair (f, f+1) an even lane stores columns (c, c+1) of register f
// and an odd lane columns (c-1, c) of register f+1, each taking the missing
// value from its neighbour.
__device__ __forceinline__ void qmm_finish_row(float (&v)[8], int lane, int colb, int row,
                                               bool live, const QmmParams& p,
                                               const float* s_svh, const float* s_bias) {
  const int n = lane & 15;
#pragma unroll
  for (int f = 0; f < 8; ++f) v[f] = round_f16(v[f]);
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
  for (int f = 0; f < 8; ++f) v[f] = bfly_lane<8>(v[f], lane);  // column stride 16: lane bit 3
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
  const bool has_bias = p.bias != nullptr;
  int cl[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    cl[f] = 32 * (f >> 1) + 16 * (n >> 3) + 8 * (f & 1) + (n & 7);
    v[f] = round_f16(round_f16(v[f] * kHadScale) * s_svh[cl[f]]);
  }
  if (p.y_dtype == DT_F32) {
    if (live) {
#pragma unroll
      for (int f = 0; f < 8; ++f)
        ((float*)p.y)[(size_t)row * p.out + colb + cl[f]] = has_bias ? v[f] + s_bias[cl[f]] : v[f];
    }
    return;
  }
  const bool odd = n & 1;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float mine = odd ? v[2 * w + 1] : v[2 * w];
    const float other = xor_lanes<1>(odd ? v[2 * w] : v[2 * w + 1]);
    const int c = cl[2 * w + (odd ? 1 : 0)];  // column of `mine`
    const int c_lo = odd ? c - 1 : c;
    const float lo = odd ? other : mine, hi = odd ? mine : other;
    const uint32_t bits = out16(lo, s_bias[c_lo], has_bias, p.y_dtype) |
                          (out16(hi, s_bias[c_lo + 1], has_bias, p.y_dtype) << 16);
    if (live) *(uint32_t*)((uint16_t*)p.y + (size_t)row * p.out + colb + c_lo) = bits;
  }
}

// Decode one step's 8 tiles of a producer (B[0] = previous lane's last word,
// B[1..K] own words) into its 4 fragments in LDS.
template <int K, int CB>
__device__ __forceinline__ void qmm_produce(const uint32_t (&B)[K + 1], u32x4* dst, int lane) {
  uint32_t src[32];
  extract_states<K>(B, src);
  dst[0 * 64 + lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 0, 0>(src));
  dst[1 * 64 + lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 0, 1>(src));
  dst[2 * 64 + lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 1, 0>(src));
  dst[3 * 64 + lane] = __builtin_bit_cast(u32x4, decode_fragment<CB, K, 1, 1>(src));
}

template <int K, int CB, int MB>
__global__ __launch_bounds__(512) void qmm_kernel(QmmParams p) {
  __shared__ u32x4 bsh[2][4][4][64];  // [buffer][producer][fragment h*2+cg][lane]
  __shared__ float s_svh[128], s_bias[128];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int role = wave & 3;
  const int TN = p.out >> 4;

  // Workgroup -> (row tile, column block, split).  Workgroups are dispatched
  // round-robin over the 8 XCDs; renumbering them so that each XCD takes a
  // contiguous range with the row tile varying slowest keeps an XCD on one
  // (or two) row tiles, whose A rows (64*MB rows x in) then stay in its L2
  // while it walks the column blocks.
  const int nwg = p.mtiles * p.col_blocks * p.splits;
  const int id = blockIdx.x;
  const int lin = (nwg & 7) == 0 ? (id & 7) * (nwg >> 3) + (id >> 3) : id;
  const int per_tile = p.col_blocks * p.splits;
  const int mtile = lin / per_tile;
  const int rest = lin - mtile * per_tile;
  const int cblk = rest % p.col_blocks, split = rest / p.col_blocks;
  const int nq_all = p.in >> 6;
  const int qa = split * nq_all / p.splits, nq = (split + 1) * nq_all / p.splits - qa;
  const int qlast = nq - 1;
  const int g = lane >> 4, n = lane & 15;
  const int tile = mtile * p.col_blocks + cblk;

  // The two roles run separate loops with the same number of barriers (one
  // per step), so their register live ranges do not overlap.
  if (wave < 4) {
    // the block's svh and bias go to LDS for the consumers' epilogue
    if (threadIdx.x < 128) {
      s_svh[threadIdx.x] = h2f(p.svh[cblk * 128 + threadIdx.x]);
      s_bias[threadIdx.x] = p.bias ? h2f(p.bias[cblk * 128 + threadIdx.x]) : 0.f;
    }
    // ---- producer: trellis slices of steps q+1..q+4 in flight ----
    constexpr int PD = 4;
    const int hsel = (lane >> 3) & 1, j = lane & 7;
    const size_t qstride = (size_t)4 * TN * 8 * K;
    const uint32_t* tp = p.trellis +
                         ((size_t)(4 * qa + g) * TN + cblk * 8 + role * 2 + hsel) * (8 * K) +
                         (size_t)j * K;
    const int prev_off = j == 0 ? 8 * K - 1 : -1;
    uint32_t sl[PD][K + 1];
#pragma unroll
    for (int d = 0; d < PD; ++d)
      load_slice_prev<K>(tp + (size_t)min(d, qlast) * qstride, prev_off, sl[d]);
    qmm_produce<K, CB>(sl[0], &bsh[0][role][0][0], lane);
    load_slice_prev<K>(tp + (size_t)min(PD, qlast) * qstride, prev_off, sl[0]);
    __syncthreads();
    // step q (phase P = q % 4): decode step q+1 from slot (q+1) % 4 into
    // buffer (q+1) & 1, refill the slot with step q+5.  Unconditional: at
    // q = nq-1 the decode lands in the buffer no consumer reads again, and the
    // loads are clamped, so the load count per step is static and the waits
    // before each decode stay partial.
    auto iter = [&](int q, auto phase) {
      constexpr int P = decltype(phase)::value;
      qmm_produce<K, CB>(sl[(P + 1) % PD], &bsh[(q + 1) & 1][role][0][0], lane);
      load_slice_prev<K>(tp + (size_t)min(q + 1 + PD, qlast) * qstride, prev_off,
                         sl[(P + 1) % PD]);
      __syncthreads();
    };
    const int nq4 = nq & ~3;
    for (int q = 0; q < nq4; q += 4) {
      iter(q, std::integral_constant<int, 0>{});
      iter(q + 1, std::integral_constant<int, 1>{});
      iter(q + 2, std::integral_constant<int, 2>{});
      iter(q + 3, std::integral_constant<int, 3>{});
    }
    if (nq4 < nq) iter(nq4, std::integral_constant<int, 0>{});
    if (nq4 + 1 < nq) iter(nq4 + 1, std::integral_constant<int, 1>{});
    if (nq4 + 2 < nq) iter(nq4 + 2, std::integral_constant<int, 2>{});
    if (p.splits > 1) {  // the arrival count of the split-K exchange below
      __syncthreads();
      if (threadIdx.x == 0) {
        uint32_t old = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == (uint32_t)(p.splits - 1));
      }
      __syncthreads();
    }
    return;
  }

  // ---- consumer: A fragments of steps q and q+1 in flight ----
  // Rows past M read row 0 (in bounds) and produce outputs that are never stored.
  const int row_base = mtile * 64 * MB + role * 16 * MB;
  const uint16_t* arow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = row_base + 16 * mb + n;
    arow[mb] = p.xhat + (size_t)(row < p.M ? row : 0) * p.in + (size_t)qa * 64 + g * 16;
  }
  half8 abuf[2][MB][2];
  auto load_a = [&](half8(&dst)[MB][2], int q) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const half8* src = (const half8*)(arow[mb] + min(q, qlast) * 64);
      dst[mb][0] = src[0];
      dst[mb][1] = src[1];
    }
  };
  float4v acc[MB][8];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int f = 0; f < 8; ++f) acc[mb][f] = float4v{0.f, 0.f, 0.f, 0.f};
  load_a(abuf[0], 0);
  load_a(abuf[1], 1);
  __syncthreads();
  // step q: multiply with A buffer q % 2, then refill it with step q+2.  The
  // B fragments of producer w2+1 are read from LDS while those of w2 feed the
  // MFMAs.
  auto iter = [&](int q, auto phase) {
    constexpr int P = decltype(phase)::value;
    half8(&a)[MB][2] = abuf[P & 1];
    const u32x4* bb = &bsh[q & 1][0][0][lane];
    half8 bc[4], bn[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) bc[f] = __builtin_bit_cast(half8, bb[f * 64]);
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      if (w2 < 3) {
#pragma unroll
        for (int f = 0; f < 4; ++f) bn[f] = __builtin_bit_cast(half8, bb[((w2 + 1) * 4 + f) * 64]);
      }
      // keep the reads of the next group ahead of this group's MFMAs
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int cg = 0; cg < 2; ++cg)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[mb][w2 * 2 + cg] = mfma16(a[mb][h], bc[h * 2 + cg], acc[mb][w2 * 2 + cg]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = 0; f < 4; ++f) bc[f] = bn[f];
    }
    load_a(a, q + 2);
    __syncthreads();
  };
  const int nq2 = nq & ~1;
  for (int q = 0; q < nq2; q += 2) {
    iter(q, std::integral_constant<int, 0>{});
    iter(q + 1, std::integral_constant<int, 1>{});
  }
  if (nq2 < nq) iter(nq2, std::integral_constant<int, 0>{});

  const int colb = cblk * 128;
  if (p.splits == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row_base + 16 * mb + 4 * g + r;
        float v[8];
#pragma unroll
        for (int f = 0; f < 8; ++f) v[f] = acc[mb][f][r];
        qmm_finish_row(v, lane, colb, row, row < p.M, p, s_svh, s_bias);
      }
    return;
  }

  // split-K: store f32 partials; the producers' thread 0 counts arrivals
  // between the two barriers; the last arriver finishes the tile
  float* part = p.partials + (size_t)split * p.M * p.out;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row_base + 16 * mb + 4 * g + r;
      if (row < p.M) {
#pragma unroll
        for (int f = 0; f < 8; ++f) {
          const int c = colb + 32 * (f >> 1) + 16 * (n >> 3) + 8 * (f & 1) + (n & 7);
          store_coherent(part + (size_t)row * p.out + c, acc[mb][f][r]);
        }
      }
    }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __syncthreads();
  if (!s_last) return;  // uniform
  if (threadIdx.x == 256)
    __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // every split's partial, this workgroup's own included, is read back from
  // memory and added in split order
#pragma unroll 1
  for (int i = 0; i < 4 * MB; ++i) {
    const int row = row_base + 16 * (i >> 2) + 4 * g + (i & 3);
    const int lrow = row < p.M ? row : p.M - 1;  // in-bounds loads for padding rows
    float v[8];
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int c = colb + 32 * (f >> 1) + 16 * (n >> 3) + 8 * (f & 1) + (n & 7);
      float sum = 0.f;
      for (int s = 0; s < p.splits; ++s)
        sum += load_coherent(p.partials + ((size_t)s * p.M + lrow) * p.out + c);
      v[f] = sum;
    }
    qmm_finish_row(v, lane, colb, row, row < p.M, p, s_svh, s_bias);
  }
}

}  // namespace exl3
