// Balanced QMV for one projection at M <= 16 rows: the whole linear
// (prologue, weight stream, cross-workgroup reduction, epilogue) in one
// launch whose decode work is split evenly over a fixed number of workgroups
// (one per CU).
//
// Work units.  A "block-step" (b, s) is 64 input rows (four tile rows, K-step
// s of NQ = in/64) of one 128-column output block b of NB = out/128: 32
// tiles, decoded by 4 waves that own two adjacent output tiles each (the
// QMV's lane ownership: one 64-lane K-dword load brings in 8 tiles, lanes
// 16g..16g+15 hold tile row 4s+g).  The V = NB * NQ block-steps are numbered
// block-major, K-step minor, and cut into VW = G * KP equal contiguous ranges,
// one per "wave group" (4 waves, one per column pair); workgroup c runs wave
// groups c*KP .. c*KP+KP-1.  Every CU decodes the same number of weights (to
// within one block-step per wave group).  A range spans at most two blocks
// (the host keeps ranges no longer than NQ).
//
// Reduction.  A wave's f32 sums of each block it touches go to the block's
// contributor slot j = (wave group) - (first wave group of the block), so a
// block receives the sums of C_b <= CMAX consecutive wave groups.  After its
// loop a workgroup counts one arrival per block it touched; in the last
// workgroup to arrive at a block one wave adds the C_b slots in slot order
// (deterministic) and runs the output epilogue (linear.rs:984-997) for the
// block's 128 columns.  The summation order depends only on the shape and the schedule
// (G, KP), never on M, so every row of a batch of M <= 16 equals the same row
// computed alone.
//
// Ordering of the exchange (agent scope, across XCDs): the slot stores are
// agent-scope relaxed atomic stores (sc1: written through to the device
// coherence point, not held in the XCD's L2); s_waitcnt vmcnt(0) in every
// wave and a workgroup barrier order all of them, acknowledged by that point,
// before the workgroup's relaxed atomic add on the block counter (also
// performed at the coherence point);
// the last arriver reads the slots with agent-scope relaxed atomic loads
// (sc1: served by the coherence point, never by a stale L1/L2 line).  So a
// slot is visible to every reader that observed the arrival that follows it.
// A release/acquire pair at agent scope adds an L2 writeback and invalidate
// (buffer_wbl2 / buffer_inv) per arrival, which measured 36 us instead of
// 24 us per launch of an earlier form of this kernel at 4096x14336.
//
// Prologue: with the fused prologue each workgroup computes
// xhat = f16(H128(f16(x) * suh) / sqrt(128)) for the 128-input blocks its
// range touches (at most two intervals of K-steps) into LDS in the order its
// steps consume them (local step u of the workgroup's range holds the 64 rows
// of its K-step), so a wave's A fragments sit at a constant stride; for larger
// batches a separate prologue launch leaves xhat in the workspace and the
// waves read their A fragments from there (PRE), one step ahead.
//
// Loads go through buffer resources: the trellis slice of a step is one scalar
// offset (computed on the scalar unit) plus per-lane offsets fixed for the
// wave, so a step costs no vector address arithmetic; loads past the end of
// the trellis read zeros.
#pragma once

#include "exl3_qmv.hpp"

namespace exl3 {

// Buffer-resource word 3 for raw (untyped, unswizzled) buffers on gfx9 parts.
constexpr int kRawBufferConfig = 0x00020000;
// Cache policy of the streamed trellis loads: nontemporal.
constexpr int kBufNt = 2;
// Column blocks one workgroup's range can touch (ranges of at most 2 NQ).
constexpr int kQmvbMaxBlocksPerWg = 3;

// One lane's slice of a tile step through a buffer resource: w[0] = the
// previous lane's last word (at loff_prev), w[1..K] the lane's K words (at
// loff), both at scalar offset soff.
template <int K>
__device__ __forceinline__ void load_slice_buf(__amdgpu_buffer_rsrc_t rs, uint32_t soff,
                                               uint32_t loff, uint32_t loff_prev,
                                               uint32_t (&w)[K + 1]) {
  w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff_prev, (int)soff, kBufNt);
  if constexpr (K == 4 || K == 8) {
#pragma unroll
    for (int h = 0; h < K / 4; ++h) {
      const u32x4 v =
          __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(loff + 16 * h), (int)soff, kBufNt);
      w[1 + 4 * h] = v[0], w[2 + 4 * h] = v[1], w[3 + 4 * h] = v[2], w[4 + 4 * h] = v[3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i)
      w[i + 1] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(loff + 4 * i), (int)soff, kBufNt);
  }
}

// Sum of a block's contributor slots for columns (lane, lane+64) of row m,
// slots added in slot order; the loads of up to kSplitChunk slots go out
// together.
__device__ __forceinline__ void qmvb_sum_row(const float* part, int C, int M, int m, int lane,
                                             float& v0, float& v1) {
  v0 = 0.f;
  v1 = 0.f;
  for (int j0 = 0; j0 < C; j0 += kSplitChunk) {
    float a[kSplitChunk], b[kSplitChunk];
#pragma unroll
    for (int i = 0; i < kSplitChunk; ++i) {
      const int jj = min(j0 + i, C - 1);  // clamped: always a written slot
      const float* ps = part + ((size_t)jj * M + m) * 128;
      a[i] = load_coherent(ps + lane);
      b[i] = load_coherent(ps + lane + 64);
    }
#pragma unroll
    for (int i = 0; i < kSplitChunk; ++i)
      if (j0 + i < C) {
        v0 += a[i];
        v1 += b[i];
      }
  }
}

// KP wave groups per workgroup (4*KP waves).  MULTI = false: one row and the
// fused prologue (the batch-1 decode).  PRE: A rows from the workspace xhat
// (separate prologue launch).
template <int K, int CB, int KP, bool PRE, bool MULTI>
__global__ __launch_bounds__(256 * KP) void qmvb_kernel(QmvParams p) {
  extern __shared__ __attribute__((aligned(16))) _Float16 xs[];  // [M][in] (fused prologue)
  // readfirstlane: the wave index is uniform, and so is everything derived
  // from it (ranges, addresses), which then stays in scalar registers
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int pair = wave & 3, part = wave >> 2;
  const Member& mm = p.mem[0];
  const int NQ = p.in >> 6, NB = mm.out >> 7, TN = mm.out >> 4;
  const int64_t V = (int64_t)NB * NQ, VW = (int64_t)gridDim.x * KP;
  const int r = blockIdx.x * KP + part;
  const int va = (int)((int64_t)r * V / VW), vb = (int)((int64_t)(r + 1) * V / VW);
  const int L = vb - va;  // block-steps of this wave (1 <= L <= NQ)
  const int M = MULTI ? p.M : 1;
  const int b0 = va / NQ, s0 = va - b0 * NQ;
  // the workgroup's range [wa, wa + NL): local step u is block-step wa + u
  const int wa = (int)((int64_t)blockIdx.x * KP * V / VW);
  const int NL = (int)((int64_t)(blockIdx.x + 1) * KP * V / VW) - wa;
  const int sw = wa % NQ;  // K-step of local step 0
  // ic: the last step of the first block; a range that crosses into block
  // b0 + 1 continues there at K-step 0
  const bool cross = s0 + L > NQ;
  const int ic = cross ? NQ - 1 - s0 : L - 1;
  __builtin_amdgcn_s_setprio(3);

  // ---- fused prologue jobs: (row, 128-input block) of the blocks this
  // workgroup's range touches, [k1, k1 + nk1) then [0, nk2) ----
  constexpr int kPro = 4;  // jobs per wave whose loads go out together
  int k1 = 0, nk1 = 0, nk2 = 0, njobs = 0;
  PrologueIn pin[kPro];
  auto job_args = [&](int jb, int& m, int& kb) {
    m = jb / (nk1 + nk2);
    const int t = jb - m * (nk1 + nk2);
    kb = t < nk1 ? k1 + t : t - nk1;
  };
  auto pro_load = [&](int j0) {
#pragma unroll
    for (int t = 0; t < kPro; ++t) {
      const int jb = min(j0 + t * 4 * KP, njobs - 1);  // clamped: always a valid job
      int m, kb;
      job_args(jb, m, kb);
      pin[t] = prologue_load(p.x, p.x_dtype, (size_t)m * p.in + kb * 128, mm.suh, kb * 128, lane);
    }
  };
  if constexpr (!PRE) {
    if (NL >= NQ) {
      nk1 = p.in >> 7;
    } else {
      const int e = sw + NL;
      k1 = sw >> 1;
      nk1 = ((min(e, NQ) + 1) >> 1) - k1;
      if (e > NQ) nk2 = min((e - NQ + 1) >> 1, k1);  // [0, nk2) stays below k1
    }
    njobs = M * (nk1 + nk2);
    pro_load(wave);  // these loads go out ahead of the weight stream
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- weight stream offsets: step i of the wave reads block-step
  // (b0, s0 + i) for i <= ic, else (b0 + 1, i - ic - 1); the byte offset is
  // (i <= ic ? off0 : off1) + i * qbytes (32-bit arithmetic, the host keeps
  // trellises below 4 GiB) ----
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7;
  const uint32_t loff = (uint32_t)(((g * TN + hsel) * 8 * K + j * K) * 4);
  const uint32_t loff_prev = loff + (uint32_t)((j == 0 ? 8 * K - 1 : -1) * 4);
  const uint32_t qbytes = (uint32_t)(128 * K * TN);  // one K-step (4 tile rows)
  const uint32_t off0 = (uint32_t)(((4 * s0) * TN + 8 * b0 + 2 * pair) * (32 * K));
  const uint32_t off1 =
      (uint32_t)((8 * (b0 + 1) + 2 * pair) * (32 * K)) - (uint32_t)(ic + 1) * qbytes;
  const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)mm.trellis, (short)0, (int)((uint32_t)(p.in / 16) * (uint32_t)TN * 32 * K),
      kRawBufferConfig);
  auto slice = [&](int i) {
    i = min(i, L - 1);  // past the end the last step is re-read (static load count)
    return (i <= ic ? off0 : off1) + (uint32_t)i * qbytes;
  };
  constexpr int D = kQmvDepth<K>;
  uint32_t setA[D][K + 1], setB[D][K + 1];
#pragma unroll
  for (int d = 0; d < D; ++d) load_slice_buf<K>(trs, slice(d), loff, loff_prev, setA[d]);
  __builtin_amdgcn_sched_barrier(0);

  // the first slices are in flight: the prologue runs meanwhile
  if constexpr (!PRE) {
    for (int j0 = wave; j0 < njobs; j0 += kPro * 4 * KP) {
      if (j0 != wave) pro_load(j0);
#pragma unroll
      for (int t = 0; t < kPro; ++t) {
        const int jb = j0 + t * 4 * KP;
        if (jb < njobs) {
          int m, kb;
          job_args(jb, m, kb);
          float v0, v1;
          prologue_finish(pin[t], p.x_dtype, lane, v0, v1);
          // K-steps 2kb (v0) and 2kb+1 (v1) at every local step that reads
          // them (one or two: the range may hold a K-step of two blocks)
          _Float16* row = xs + (size_t)m * NL * 64;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int u = (2 * kb + h - sw + NQ) % NQ;
            const _Float16 v = (_Float16)(h ? v1 : v0);
            if (u < NL) row[u * 64 + lane] = v;
            if (u + NQ < NL) row[(u + NQ) * 64 + lane] = v;
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- main loop: two sets of D slices in ping-pong (as the QMV) ----
  // A rows >= M read row M-1: MFMA output rows depend only on their own A row
  // and rows >= M are never stored.
  const int am = min(lane & 15, M - 1);
  // fused: the wave's step i is local step (va - wa) + i
  const _Float16* xa = xs + (size_t)am * NL * 64 + (va - wa) * 64 + g * 16;
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  float4v fin0 = acc0, fin1 = acc1;  // sums of block b0 when the range crosses
  const int t1 = (L + 3) / 4, t2 = (2 * L + 3) / 4, t3 = (3 * L + 3) / 4;
  // PRE: the A fragments of a step, loaded one step ahead (byte offset of
  // K-step kstep(i) = (i <= ic ? s0 : -(ic + 1)) + i, times 128)
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)mm.xhat, (short)0, (int)((uint32_t)M * p.in * 2), kRawBufferConfig);
  const uint32_t xoff = (uint32_t)((am * p.in + g * 16) * 2);
  auto load_a = [&](int i, u32x4(&dst)[2]) {
    const uint32_t so = ((uint32_t)(i <= ic ? s0 : -(ic + 1)) + (uint32_t)i) * 128u;
    dst[0] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)xoff, (int)so, 0);
    dst[1] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)(xoff + 16), (int)so, 0);
  };
  u32x4 apre[2];
  if constexpr (PRE) load_a(0, apre);
  auto compute = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = qbase + d;
      if (i < L) {
        half8 a0, a1;
        if constexpr (PRE) {
          a0 = __builtin_bit_cast(half8, apre[0]);
          a1 = __builtin_bit_cast(half8, apre[1]);
          load_a(min(i + 1, L - 1), apre);
        } else {
          a0 = *(const half8*)(xa + i * 64);
          a1 = *(const half8*)(xa + i * 64 + 8);
        }
        qmv_step_prev<K, CB>(set[d], a0, a1, acc0, acc1);
        const int t = i + 1;
        if (t == t3) __builtin_amdgcn_s_setprio(0);
        else if (t == t2) __builtin_amdgcn_s_setprio(1);
        else if (t == t1) __builtin_amdgcn_s_setprio(2);
        if (cross && i == ic) {  // block b0 ends: keep its sums, start b0 + 1
          fin0 = acc0;
          fin1 = acc1;
          acc0 = float4v{0.f, 0.f, 0.f, 0.f};
          acc1 = float4v{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  };
  auto fetch = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d) load_slice_buf<K>(trs, slice(qbase + d), loff, loff_prev, set[d]);
  };
  for (int q0 = 0; q0 < L; q0 += 2 * D) {
    fetch(setB, q0 + D);
    compute(setA, q0);
    fetch(setA, q0 + 2 * D);
    compute(setB, q0 + D);
  }

  // ---- slots: this wave's sums of each block it touched ----
  const int CMAX = p.slots;
  const int n = lane & 15;
  const int col = 16 * (pair * 2 + (n >> 3)) + (n & 7);  // column inside the block (cg = 0)
  auto store_slot = [&](int b, const float4v& s0v, const float4v& s1v) {
    const int jslot = r - qmvb_group_of((int64_t)b * NQ, V, VW);
    float* dst = p.partials + ((size_t)b * CMAX + jslot) * M * 128 + col;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = 4 * g + q;
      if (m < M) {
        store_coherent(dst + (size_t)m * 128, s0v[q]);
        store_coherent(dst + (size_t)m * 128 + 8, s1v[q]);
      }
    }
  };
  if (cross) {
    store_slot(b0, fin0, fin1);
    store_slot(b0 + 1, acc0, acc1);
  } else {
    store_slot(b0, acc0, acc1);
  }
  __builtin_amdgcn_s_waitcnt(0);  // every slot store acknowledged (see the header)
  __syncthreads();

  // ---- arrivals, one per (workgroup, block it touched): the last workgroup
  // to arrive at a block finishes it, wave i taking the i-th block ----
  __shared__ int s_last[kQmvbMaxBlocksPerWg];
  const int G = gridDim.x;
  const int wb0 = wa / NQ, nblk = (wa + NL - 1) / NQ - wb0 + 1;  // <= 3 (NL <= 2 NQ)
  if (threadIdx.x < nblk) {
    const int b = wb0 + threadIdx.x;
    const int wgs = qmvb_group_of((int64_t)b * NQ + NQ - 1, V, G) -
                    qmvb_group_of((int64_t)b * NQ, V, G) + 1;
    const uint32_t old = __hip_atomic_fetch_add(&p.counters[b], 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    s_last[threadIdx.x] = old == (uint32_t)(wgs - 1);
    if (old == (uint32_t)(wgs - 1))
      __hip_atomic_store(&p.counters[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (wave >= nblk || !s_last[wave]) return;  // uniform across the wave
  const int b = wb0 + wave;
  const int C = qmvb_group_of((int64_t)b * NQ + NQ - 1, V, VW) -
                qmvb_group_of((int64_t)b * NQ, V, VW) + 1;
  const float* slots = p.partials + (size_t)b * CMAX * M * 128;
  for (int m = 0; m < M; ++m) {
    float v0, v1;
    qmvb_sum_row(slots, C, M, m, lane, v0, v1);
    finish_row128(v0, v1, lane, b * 128, mm.svh, mm.bias, mm.y, mm.y_dtype, p.x_dtype,
                  (size_t)m * mm.out);
  }
}

}  // namespace exl3
