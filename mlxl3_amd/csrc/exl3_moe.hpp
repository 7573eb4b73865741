// MoE SwitchGLU over EXL3 expert banks: the reference's Exl3SwitchGlu
// (native/src/moe.rs:611-1085) -- route plan, routed inputs, expert QMMs,
// SwiGLU glue, down projection, weighted top-k reduction -- re-designed for
// gfx950 as five launches:
//   1. plan:    one workgroup counting-sorts the rows*top_k slots by expert and
//               cuts each expert's run into <= 64-row blocks (block table);
//   2. gather:  f16(x[token] * gu_suh[e][p]) -> staged Hadamard-128 for the gate
//               (p = 0) and up (p = 1) inputs, in expert-sorted order;
//   3. gate/up: per (block, 128 hidden columns) a workgroup decodes the expert's
//               gate AND up tiles of those columns in registers (waves own column
//               pairs, as in the QMV) and multiplies them with the block's rows;
//               the epilogue is the whole of glu_down_input (moe.rs:435-563): f16,
//               f32 Hadamard, *scale*svh, SiLU(g)*u, *down_suh, f32 Hadamard,
//               *scale -> the down projection's xhat;
//   4. down:    same kernel shape over the down bank; the epilogue is
//               finish_and_reduce's per-slot part (moe.rs:586-609): f16, staged
//               Hadamard, *svh, *score, stored per slot;
//   5. reduce:  y[row] = f16(sum over top_k in slot order, f32).
// Each row's arithmetic is independent of the other rows of its block, so the
// (atomics-ordered) placement of slots inside an expert's run cannot change any
// result.
#pragma once

#include "exl3_device.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {

constexpr int kMoeBlockRows = 64;  // rows per block-table entry (moe.rs:80-83)

struct MoePlanParams {
  const uint32_t* selected;  // [slots] expert ids (rows * top_k)
  int slots, experts;
  int* rank;                 // [slots] scratch
  int* sorted_slot;          // [slots] slot at each sorted position
  int4* table;               // [max_blocks] (expert, first sorted position, rows, 0)
  int* counts;               // [2]: block-table entries, routed slots
  int* expert_count;         // [experts] (rows routed to each expert)
};

// One workgroup of 1024 threads.  Slots with an expert id >= experts are left
// out (their contribution is zero).
__global__ __launch_bounds__(1024) void moe_plan_kernel(MoePlanParams p) {
  extern __shared__ int lds[];  // cnt[E], off[E], boff[E+1]
  int* cnt = lds;
  int* off = lds + p.experts;
  int* boff = lds + 2 * p.experts;
  const int tid = threadIdx.x;
  for (int e = tid; e < p.experts; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int s = tid; s < p.slots; s += 1024) {
    const uint32_t e = p.selected[s];
    p.rank[s] = e < (uint32_t)p.experts ? atomicAdd(&cnt[e], 1) : -1;
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0, bacc = 0;
    for (int e = 0; e < p.experts; ++e) {
      off[e] = acc;
      boff[e] = bacc;
      acc += cnt[e];
      bacc += (cnt[e] + kMoeBlockRows - 1) / kMoeBlockRows;
    }
    boff[p.experts] = bacc;
    p.counts[0] = bacc;
    p.counts[1] = acc;
  }
  __syncthreads();
  for (int s = tid; s < p.slots; s += 1024) {
    const int r = p.rank[s];
    if (r >= 0) p.sorted_slot[off[p.selected[s]] + r] = s;
  }
  for (int e = tid; e < p.experts; e += 1024) {
    p.expert_count[e] = cnt[e];
    for (int b = boff[e]; b < boff[e + 1]; ++b) {
      const int first = off[e] + (b - boff[e]) * kMoeBlockRows;
      p.table[b] = make_int4(e, first, min(kMoeBlockRows, off[e] + cnt[e] - first), 0);
    }
  }
}

// Gate/up inputs in sorted order: xgu[proj][pos][in] with proj 0 = gate,
// 1 = up (routed_inputs, moe.rs:184-250).  grid (slots, in/128, 2), one wave
// per (block, position, projection); positions past the routed count idle.
__global__ __launch_bounds__(64) void moe_gather_kernel(const uint16_t* __restrict__ x, int in,
                                                        int top_k, const uint32_t* selected,
                                                        const int* sorted_slot,
                                                        const int* routed,
                                                        const uint16_t* __restrict__ gu_suh,
                                                        uint16_t* __restrict__ xgu) {
  const int lane = threadIdx.x, pos = blockIdx.x, b = blockIdx.y, proj = blockIdx.z;
  if (pos >= *routed) return;
  const int slot = sorted_slot[pos];
  const int token = slot / top_k;
  const uint32_t e = selected[slot];
  const uint16_t* suh = gu_suh + ((size_t)e * 2 + proj) * in;
  float v0, v1;
  prepare_row128(x, DT_F16, (size_t)token * in + b * 128, suh, b * 128, lane, v0, v1);
  uint16_t* dst = xgu + ((size_t)proj * gridDim.x + pos) * in + b * 128;
  dst[lane] = f2h(v0);
  dst[lane + 64] = f2h(v1);
}

struct MoeQmmParams {
  const uint32_t* trellis;  // bank, [K_in/16][tn_total][8K] u32
  int tn_total;             // tile columns of the bank
  int k_in;                 // input width of the projection (rows of the trellis)
  int width;                // output width of one expert's projection
  int experts;
  const int4* table;
  const int* counts;        // [0] = block-table entries
  const int* sorted_slot;
  int max_blocks;
  int col_blocks;           // width / 128
  int slots_pad;            // position stride of xgu
  // gate/up
  const uint16_t* xgu;      // [2][slots_pad][k_in]
  const uint16_t* gu_svh;   // [E][2][width]
  const uint16_t* down_suh; // [E][width]
  uint16_t* xd;             // [slots_pad][width]
  // down
  const uint16_t* xin;      // [slots_pad][k_in]
  const uint16_t* down_svh; // [E][width]
  const uint16_t* scores;   // [slots]
  uint16_t* z;              // [slots][width]
  const uint32_t* selected;
};

// One weight step of a grouped QMM: decode the wave's 8 tiles (2 output tiles x
// 4 tile rows) of `B` and run MBLK 16-row MFMA blocks against A fragments read
// from `arow` rows (row stride `k_in`), rows >= nrows contributing zero.
template <int K, int CB, int MBLK>
__device__ __forceinline__ void moe_step(const uint32_t (&B)[K + 1],
                                         const uint16_t* const (&arow)[MBLK],
                                         const bool (&aval)[MBLK], int mblocks, int q,
                                         float4v (&acc0)[MBLK], float4v (&acc1)[MBLK]) {
  uint32_t src[32];
  extract_states<K>(B, src);
  const half8 b00 = decode_fragment<CB, K, 0, 0>(src);
  const half8 b01 = decode_fragment<CB, K, 0, 1>(src);
  const half8 b10 = decode_fragment<CB, K, 1, 0>(src);
  const half8 b11 = decode_fragment<CB, K, 1, 1>(src);
  const half8 zero8 = {};
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb) {
    if (mb < mblocks) {
      // rows past the block's end read a valid row and are zeroed afterwards
      const half8* src8 = (const half8*)(arow[mb] + q * 64);
      half8 a0 = src8[0], a1 = src8[1];
      a0 = aval[mb] ? a0 : zero8;
      a1 = aval[mb] ? a1 : zero8;
      acc0[mb] = mfma16(a0, b00, acc0[mb]);
      acc1[mb] = mfma16(a0, b01, acc1[mb]);
      acc0[mb] = mfma16(a1, b10, acc0[mb]);
      acc1[mb] = mfma16(a1, b11, acc1[mb]);
    }
  }
}

// Accumulators of a wave -> LDS rows [16*mb + row][32*wave + col] (f32).
template <int MBLK>
__device__ __forceinline__ void moe_park(float* red, int wave, int lane, int mb,
                                         const float4v (&acc0)[MBLK],
                                         const float4v (&acc1)[MBLK]) {
  const int g = lane >> 4, n = lane & 15;
  const int col = 32 * wave + 16 * (n >> 3) + (n & 7);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    red[(4 * g + r) * 128 + col] = acc0[mb][r];
    red[(4 * g + r) * 128 + col + 8] = acc1[mb][r];
  }
}

// Gate/up grouped QMM with the fused SwiGLU / down-prologue epilogue.
template <int K, int CB>
__global__ __launch_bounds__(256) void moe_gateup_kernel(MoeQmmParams p) {
  constexpr int MBLK = kMoeBlockRows / 16;
  __shared__ float red[2][16 * 128];  // gate, up rows of one 16-row block
  const int blk = blockIdx.x / p.col_blocks, cblk = blockIdx.x % p.col_blocks;
  if (blk >= p.counts[0]) return;  // uniform
  const int4 ent = p.table[blk];
  const int e = ent.x, pos0 = ent.y, nrows = ent.z;
  const int mblocks = (nrows + 15) / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7, am = lane & 15;
  const int nq = p.k_in >> 6;
  const size_t qstride = (size_t)4 * p.tn_total * 8 * K;
  const int tiles_per_expert = p.width / 16;
  const int tcol = cblk * 8 + 2 * wave + hsel;
  const uint32_t* tg = p.trellis + ((size_t)g * p.tn_total + (size_t)e * tiles_per_expert + tcol) *
                                       (8 * K) + (size_t)j * K;
  const uint32_t* tu = tg + (size_t)p.experts * tiles_per_expert * (8 * K);
  const int prev_off = j == 0 ? 8 * K - 1 : -1;

  const uint16_t* ag[MBLK];
  const uint16_t* au[MBLK];
  bool aval[MBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb) {
    const int r = 16 * mb + am;
    aval[mb] = r < nrows;
    const int pos = pos0 + (aval[mb] ? r : 0);
    ag[mb] = p.xgu + (size_t)pos * p.k_in + g * 16;
    au[mb] = p.xgu + ((size_t)p.slots_pad + pos) * p.k_in + g * 16;
  }
  float4v gacc0[MBLK], gacc1[MBLK], uacc0[MBLK], uacc1[MBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb)
    gacc0[mb] = gacc1[mb] = uacc0[mb] = uacc1[mb] = float4v{0.f, 0.f, 0.f, 0.f};

  uint32_t wg[K + 1], wu[K + 1];
  load_slice_prev<K>(tg, prev_off, wg);
  load_slice_prev<K>(tu, prev_off, wu);
  for (int q = 0; q < nq; ++q) {
    uint32_t cg[K + 1], cu[K + 1];
#pragma unroll
    for (int i = 0; i <= K; ++i) cg[i] = wg[i], cu[i] = wu[i];
    const int qn = min(q + 1, nq - 1);
    load_slice_prev<K>(tg + (size_t)qn * qstride, prev_off, wg);
    load_slice_prev<K>(tu + (size_t)qn * qstride, prev_off, wu);
    moe_step<K, CB, MBLK>(cg, ag, aval, mblocks, q, gacc0, gacc1);
    moe_step<K, CB, MBLK>(cu, au, aval, mblocks, q, uacc0, uacc1);
  }

  // epilogue, one 16-row block at a time through LDS
  const int col0 = cblk * 128;
  for (int mb = 0; mb < MBLK; ++mb) {
    if (mb >= mblocks) break;  // uniform
    __syncthreads();
    moe_park<MBLK>(red[0], wave, lane, mb, gacc0, gacc1);
    moe_park<MBLK>(red[1], wave, lane, mb, uacc0, uacc1);
    __syncthreads();
    for (int r = wave; r < 16; r += 4) {
      const int row = 16 * mb + r;
      if (row >= nrows) break;
      const int pos = pos0 + row;
      // gate and up: f16(raw) -> f32 Hadamard -> f16(v * scale * svh)
      float g0 = round_f16(red[0][r * 128 + lane]), g1 = round_f16(red[0][r * 128 + lane + 64]);
      float u0 = round_f16(red[1][r * 128 + lane]), u1 = round_f16(red[1][r * 128 + lane + 64]);
      h128_wave<false>(g0, g1, lane);
      h128_wave<false>(u0, u1, lane);
      const uint16_t* gsv = p.gu_svh + ((size_t)e * 2) * p.width + col0;
      const uint16_t* usv = gsv + p.width;
      g0 = round_f16(g0 * kHadScale * h2f(gsv[lane]));
      g1 = round_f16(g1 * kHadScale * h2f(gsv[lane + 64]));
      u0 = round_f16(u0 * kHadScale * h2f(usv[lane]));
      u1 = round_f16(u1 * kHadScale * h2f(usv[lane + 64]));
      // SiLU(g) * u, then * down_suh, f32 Hadamard, f16(v * scale)
      const float a0 = round_f16((g0 / (1.0f + expf(-g0))) * u0);
      const float a1 = round_f16((g1 / (1.0f + expf(-g1))) * u1);
      const uint16_t* dsu = p.down_suh + (size_t)e * p.width + col0;
      float d0 = round_f16(a0 * h2f(dsu[lane])), d1 = round_f16(a1 * h2f(dsu[lane + 64]));
      h128_wave<false>(d0, d1, lane);
      uint16_t* dst = p.xd + (size_t)pos * p.width + col0;
      dst[lane] = f2h(d0 * kHadScale);
      dst[lane + 64] = f2h(d1 * kHadScale);
    }
  }
}

// Down grouped QMM with finish_and_reduce's per-slot epilogue.
template <int K, int CB>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeQmmParams p) {
  constexpr int MBLK = kMoeBlockRows / 16;
  __shared__ float red[16 * 128];
  const int blk = blockIdx.x / p.col_blocks, cblk = blockIdx.x % p.col_blocks;
  if (blk >= p.counts[0]) return;  // uniform
  const int4 ent = p.table[blk];
  const int e = ent.x, pos0 = ent.y, nrows = ent.z;
  const int mblocks = (nrows + 15) / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7, am = lane & 15;
  const int nq = p.k_in >> 6;
  const size_t qstride = (size_t)4 * p.tn_total * 8 * K;
  const int tiles_per_expert = p.width / 16;
  const int tcol = cblk * 8 + 2 * wave + hsel;
  const uint32_t* tp = p.trellis + ((size_t)g * p.tn_total + (size_t)e * tiles_per_expert + tcol) *
                                       (8 * K) + (size_t)j * K;
  const int prev_off = j == 0 ? 8 * K - 1 : -1;

  const uint16_t* ar[MBLK];
  bool aval[MBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb) {
    const int r = 16 * mb + am;
    aval[mb] = r < nrows;
    ar[mb] = p.xin + (size_t)(pos0 + (aval[mb] ? r : 0)) * p.k_in + g * 16;
  }
  float4v acc0[MBLK], acc1[MBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb) acc0[mb] = acc1[mb] = float4v{0.f, 0.f, 0.f, 0.f};

  uint32_t w[K + 1];
  load_slice_prev<K>(tp, prev_off, w);
  for (int q = 0; q < nq; ++q) {
    uint32_t c[K + 1];
#pragma unroll
    for (int i = 0; i <= K; ++i) c[i] = w[i];
    load_slice_prev<K>(tp + (size_t)min(q + 1, nq - 1) * qstride, prev_off, w);
    moe_step<K, CB, MBLK>(c, ar, aval, mblocks, q, acc0, acc1);
  }

  const int col0 = cblk * 128;
  for (int mb = 0; mb < MBLK; ++mb) {
    if (mb >= mblocks) break;  // uniform
    __syncthreads();
    moe_park<MBLK>(red, wave, lane, mb, acc0, acc1);
    __syncthreads();
    for (int r = wave; r < 16; r += 4) {
      const int row = 16 * mb + r;
      if (row >= nrows) break;
      const int slot = p.sorted_slot[pos0 + row];
      float v0 = round_f16(red[r * 128 + lane]), v1 = round_f16(red[r * 128 + lane + 64]);
      h128_wave<true>(v0, v1, lane);
      v0 = round_f16(v0 * kHadScale);
      v1 = round_f16(v1 * kHadScale);
      const uint16_t* sv = p.down_svh + (size_t)e * p.width + col0;
      const float sc = h2f(p.scores[slot]);
      v0 = round_f16(round_f16(v0 * h2f(sv[lane])) * sc);
      v1 = round_f16(round_f16(v1 * h2f(sv[lane + 64])) * sc);
      uint16_t* dst = p.z + (size_t)slot * p.width + col0;
      dst[lane] = f2h(v0);
      dst[lane + 64] = f2h(v1);
    }
  }
}

// y[row][i] = f16(sum_t f32(z[row*top_k + t][i])) in t order; slots routed to
// no valid expert contribute zero.  grid (rows, ceil(width/256)).
__global__ __launch_bounds__(256) void moe_reduce_kernel(const uint16_t* __restrict__ z,
                                                         const uint32_t* __restrict__ selected,
                                                         int experts, int top_k, int width,
                                                         uint16_t* __restrict__ y) {
  const int i = blockIdx.y * 256 + threadIdx.x, row = blockIdx.x;
  if (i >= width) return;
  float acc = 0.f;
  for (int t = 0; t < top_k; ++t) {
    const int slot = row * top_k + t;
    if (selected[slot] < (uint32_t)experts) acc += h2f(z[(size_t)slot * width + i]);
  }
  y[(size_t)row * width + i] = f2h(acc);
}

}  // namespace exl3
