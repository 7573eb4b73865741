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
//    fragment order (one ds_write_b128 per fragment, conflict-free), and
//    copies consumer w's A rows (xhat) into LDS; trellis slices are loaded
//    four steps ahead, A rows two;
//  * consumer w owns 16*MB rows and multiplies them by all 16 fragments of the
//    step, reading the next fragment group while the current group's MFMAs
//    issue.
// Three LDS stages and one workgroup barrier per step: producers fill step
// q+2 while consumers multiply step q.  Each weight is decoded once per 64*MB
// rows.
//
// After the loop the consumers round their accumulators to f16 rows in LDS and
// all 8 waves run the output epilogue (f16 -> staged H128 -> * svh -> cast,
// linear.rs:1940-1963) with 8 consecutive columns per lane.  With a global
// split-K the K-ranges leave f32 partials (exchanged with agent-scope relaxed
// atomics, as in the QMV) and the last workgroup of an output tile adds them
// in split order, so results do not depend on timing.
#pragma once

#include "exl3_device.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {

// xhat[i] = prologue(x, suh[i]) for all rows of each member i (grid.y), 16
// lanes per (row, 128-block) job (prologue8).  suh_stride = in gives every
// row its own scales (exl3_prepare128).  grid (ceil(rows * blocks / 16),
// members), 256 threads.
// The (row, 128-block) job of this lane's DPP row when each workgroup of 256
// threads takes 16 consecutive jobs of a rows x nb grid; returns whether the
// job exists.  Past-the-end jobs become the last one (all lanes of a DPP row
// stay active) and are not stored.  The workgroup's first job is divided once,
// uniformly and in 32 bits (rows * nb < 2^24: the entry points reject
// rows * in > INT32_MAX); a lane's job lies at most 15 blocks further, so rows
// advance by subtraction (at most once when a row has 16 blocks or more).
__device__ __forceinline__ bool job16(int rows, int nb, int& row, int& b) {
  const uint32_t n = (uint32_t)nb, j0 = blockIdx.x * 16u;
  const uint32_t row0 = j0 / n;
  uint32_t bu = j0 - row0 * n + (threadIdx.x >> 4), ru = row0;
  while (bu >= n) {
    bu -= n;
    ++ru;
  }
  const bool live = ru < (uint32_t)rows;
  row = live ? (int)ru : rows - 1;
  b = live ? (int)bu : nb - 1;
  return live;
}

template <bool VEC>
__global__ __launch_bounds__(256) void prologue_kernel(PrologueParams p) {
  int row, b;
  const bool live = job16(p.rows, p.in >> 7, row, b);
  const int c8 = 8 * (threadIdx.x & 15);
  const uint16_t* suh = p.suh[0];
  uint16_t* xhat = p.xhat[0];
#pragma unroll
  for (int i = 1; i < kMaxMembers; ++i)
    if ((int)blockIdx.y == i) {
      suh = p.suh[i];
      xhat = p.xhat[i];
    }
  const size_t e = (size_t)row * p.in + (size_t)b * 128 + c8;
  prologue8<VEC>(p.x, p.x_dtype, e, suh + (size_t)row * p.suh_stride + (size_t)b * 128 + c8,
                 xhat + e, live, threadIdx.x & 63);
}

// The SwiGLU edge between a (gate, up) group and its down projection:
// xhat_down = f16(H128(f16(swiglu(g, u) * down_suh)) / sqrt(128)) (the down
// projection's prologue applied to the activation, as the reference's
// flash_up_finish_swiglu_prepare fuses them, exl3.metal:265-291, with
// Array::swiglu's f16 arithmetic).  16 lanes per (row, 128-block) job, 8
// columns per lane (finish8).  grid (ceil(rows * H / 128 / 16)), 256 threads.
template <bool VEC>
__global__ __launch_bounds__(256) void swiglu_prepare_kernel(const uint16_t* __restrict__ gate,
                                                             const uint16_t* __restrict__ up,
                                                             const uint16_t* __restrict__ down_suh,
                                                             int H, int rows,
                                                             uint16_t* __restrict__ xhat) {
  int row, b;
  const bool live = job16(rows, H >> 7, row, b);
  const int c = b * 128 + 8 * (threadIdx.x & 15);
  const size_t e = (size_t)row * H + c;
  float a[8], sv[8];
  if constexpr (VEC) {
    const u32x4 gw = *(const u32x4*)(gate + e), uw = *(const u32x4*)(up + e);
    const u32x4 sw = *(const u32x4*)(down_suh + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = swiglu_f16(h2f((uint16_t)gw[i]), h2f((uint16_t)uw[i]));
      a[2 * i + 1] = swiglu_f16(h2f((uint16_t)(gw[i] >> 16)), h2f((uint16_t)(uw[i] >> 16)));
      sv[2 * i] = h2f((uint16_t)sw[i]);
      sv[2 * i + 1] = h2f((uint16_t)(sw[i] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = swiglu_f16(h2f(gate[e + i]), h2f(up[e + i]));
      sv[i] = h2f(down_suh[c + i]);
    }
  }
  finish8<VEC>(a, sv, xhat + e, live, threadIdx.x & 63);
}

// Rows of a finished tile pass through LDS as f16: Y[row][136] (128 columns
// plus 8 halves of padding, so the 16-byte reads of one row never meet the
// next row's banks).
constexpr int kYStride = 136;

// Consumer side: f16(acc) of one row into Y.  Register f of the lane holds
// column 32*(f>>1) + 8*(f&1) + lanecol, lanecol = 16*(n>>3) + (n&7), n =
// lane & 15.  Neighbouring lanes swap one value so that each lane writes two
// 32-bit column pairs: an even lane columns (c, c+1) of register 2w, an odd
// lane columns (c-1, c) of register 2w+1.
__device__ __forceinline__ void qmm_stage_row(const float (&v)[8], int lane, uint16_t* yrow) {
  const int n = lane & 15;
  const bool odd = n & 1;
  const int pcol = 16 * (n >> 3) + (n & 7) + (odd ? 7 : 0);
  uint32_t* y32 = (uint32_t*)(yrow + pcol);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float mine = odd ? v[2 * w + 1] : v[2 * w];
    const float other = xor_lanes<1>(odd ? v[2 * w] : v[2 * w + 1]);
    const float lo = odd ? other : mine, hi = odd ? mine : other;
    y32[16 * w] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
  }
}

// Value of the linear epilogue's final cast (+ bias), as out_value computes
// it: the cast to the activation dtype x_dt, then the bias added with MLX's
// promotion (f16 + f16 in f16, f32 or bf16 + f16 in f32).
__device__ __forceinline__ float out_cast(float v16, float b, bool has_bias, int x_dt) {
  float v = x_dt == DT_BF16 ? bf2f(f2bf(v16)) : v16;
  if (has_bias) v = x_dt == DT_F16 ? round_f16(v + b) : v + b;
  return v;
}
// 16-bit output bits (f16 or bf16 result dtype).
__device__ __forceinline__ uint32_t out16(float v, int y_dt) {
  return y_dt == DT_F16 ? f2h(v) : f2bf(v);
}

// Finishing side: each lane holds 8 consecutive columns 8*(lane&15)+j of one
// row (four rows per wave pass): f16 values -> staged Hadamard-128 (strides
// 1, 2, 4 inside the lane, 8..64 across lanes 1..8, f16 rounding after
// strides 8 and 64) -> f16(* 1/sqrt 128) -> f16(* svh) -> cast (+ bias) ->
// one 16-byte store (two for f32).  sv/bv: svh and bias of the lane's columns.
__device__ __forceinline__ void qmm_finish_chunk(const u32x4 raw, const float (&sv)[8],
                                                 const float (&bv)[8], int lane, bool live,
                                                 const Member& mm, int x_dtype, size_t yoff) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f((uint16_t)raw[i]);
    v[2 * i + 1] = h2f((uint16_t)(raw[i] >> 16));
  }
  h128_lane8(v, lane);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = round_f16(round_f16(v[j] * kHadScale) * sv[j]);
  if (!live) return;
  const bool has_bias = mm.bias != nullptr;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = out_cast(v[j], bv[j], has_bias, x_dtype);
  if (mm.y_dtype == DT_F32) {
    float4v o0, o1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o0[j] = v[j];
      o1[j] = v[j + 4];
    }
    float4v* yp = (float4v*)((float*)mm.y + yoff);
    yp[0] = o0;
    yp[1] = o1;
    return;
  }
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = out16(v[2 * i], mm.y_dtype) | (out16(v[2 * i + 1], mm.y_dtype) << 16);
  *(u32x4*)((uint16_t*)mm.y + yoff) = o;
}

// load_slice_prev<K> as raw buffer loads with a fixed count of load
// instructions, 2 for K <= 4 and 3 above (the previous lane's word, then the
// lane's K words as 1-4 word loads at 4-byte alignment), which the producers'
// direct A copies wait around: resource `r`, the step's scalar byte offset
// `so`, the lane's byte offsets of its words (`lo`) and of the previous lane's
// last word (`lo_prev`).
template <int K>
constexpr int kSliceLoads = K <= 4 ? 2 : 3;
template <int N>
__device__ __forceinline__ void buffer_words(__amdgpu_buffer_rsrc_t r, uint32_t lo, uint32_t so,
                                             uint32_t* w) {
  if constexpr (N == 1) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, lo, so, kCpolNt);
  } else if constexpr (N == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, lo, so, kCpolNt);
    w[0] = v[0], w[1] = v[1];
  } else if constexpr (N == 3) {
    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, lo, so, kCpolNt);
    w[0] = v[0], w[1] = v[1], w[2] = v[2];
  } else {
    static_assert(N == 4, "1-4 words");
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, lo, so, kCpolNt);
    w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
  }
}
template <int K>
__device__ __forceinline__ void buffer_slice_counted(__amdgpu_buffer_rsrc_t r, uint32_t so,
                                                     uint32_t lo, uint32_t lo_prev,
                                                     uint32_t (&w)[K + 1]) {
  w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, lo_prev, so, kCpolNt);
  buffer_words<(K < 4 ? K : 4)>(r, lo, so, w + 1);
  if constexpr (K > 4) buffer_words<K - 4>(r, lo + 16, so, w + 5);
}

// Buffer resource over the split-K partials of (split, tile): the f32
// accumulators of the tile's 4 consumers in fragment order, [consumer][mb][f]
// [lane] of 16 bytes (MB * 32 KB).
template <class P>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t qmm_slab(const P& p, int split, int tile,
                                                          int MB) {
  return __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.partials + ((size_t)split * p.mtiles * p.col_blocks + tile) * (MB * 8192)), 0,
      MB * 32768, kBufferRsrcWord3);
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
  // LDS: three stages of B fragments (16 KB each) and of A rows (64*MB rows x
  // 128 bytes each), as two objects so that the compiler can tell the A
  // stages' direct loads from the B stores (no wait for the loads before
  // those); after the K loop the A bytes hold the tile's f16 rows.
  constexpr int kBStage = 16384, kAStage = 64 * MB * 128;
  constexpr int kY = 64 * MB * kYStride * 2;
  constexpr int kABytes = 3 * kAStage > kY ? 3 * kAStage : kY;
  __shared__ __attribute__((aligned(16))) uint8_t bls[3 * kBStage];
  __shared__ __attribute__((aligned(16))) uint8_t als[kABytes];
  uint16_t* ys = (uint16_t*)als;  // [64*MB][kYStride] after the loop
  __shared__ float s_svh[128], s_bias[128];
  __shared__ int s_last;
  auto bstage = [&](int st) { return (u32x4*)(bls + st * kBStage); };  // [producer][frag][lane]
  auto astage = [&](int st) { return als + st * kAStage; };

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int role = wave & 3;

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
  const int cblk = rest % p.col_blocks, split = rest / p.col_blocks;  // global column block
  const Member mm = select_member(p, cblk);
  const int cblk_l = cblk - mm.cblk0;  // column block inside the member
  const int TN = mm.out >> 4;
  const int TO = p.total_out;
  const int nq_all = p.in >> 6;
  const int qa = split * nq_all / p.splits, nq = (split + 1) * nq_all / p.splits - qa;
  const int qlast = nq - 1;
  const int g = lane >> 4, n = lane & 15;
  const int tile = mtile * p.col_blocks + cblk;
  const int row_base = mtile * 64 * MB + role * 16 * MB;  // first row of consumer `role`

  // A rows sit in LDS as [row][8 chunks of 16 bytes] with chunk c of row r at
  // slot c ^ a_swizzle(r): the producers' row-wise writes and the
  // consumers' fragment reads (16 rows x one chunk) are both free of bank
  // conflicts.

  // Step s of the K loop uses stage s % 3.  In iteration q the producers fill
  // stage (q+2) % 3 with step q+2 while the consumers multiply step q and,
  // before the barrier, read the first fragments of step q+1 (written in
  // iteration q-1).  One barrier per iteration orders both.
  if (wave < 4) {
    // ---- producer `role`: B tiles of output tiles 2*role, 2*role+1 and the
    // A rows of consumer `role` ----
    if (threadIdx.x < 128) {
      s_svh[threadIdx.x] = h2f(mm.svh[cblk_l * 128 + threadIdx.x]);
      s_bias[threadIdx.x] = mm.bias ? h2f(mm.bias[cblk_l * 128 + threadIdx.x]) : 0.f;
    }
    // trellis slices in flight: 4 steps ahead (with A copied straight to LDS
    // at MB >= 2 no variant spills at this depth)
    constexpr int PD = 4;
    const int hsel = (lane >> 3) & 1, j = lane & 7;
    const size_t qstride = (size_t)4 * TN * 8 * K;
    const uint32_t* tp = mm.trellis +
                         ((size_t)(4 * qa + g) * TN + cblk_l * 8 + role * 2 + hsel) * (8 * K) +
                         (size_t)j * K;
    const int prev_off = j == 0 ? 8 * K - 1 : -1;
    // With the direct A copies the slices are raw buffer loads from the
    // workgroup's base (its first quad and column block: uniform, held in
    // scalar registers, bounded by the end of the member's trellis): the
    // producer's and the lane's parts sit in the 32-bit vector offset, the
    // step's in the scalar one, so a slice costs no vector address work.
    const size_t wg_words = ((size_t)4 * qa * TN + cblk_l * 8) * (8 * K);
    const size_t tensor_words = (size_t)(p.in >> 4) * TN * (8 * K);
    const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(mm.trellis + wg_words), 0,
        (int)(uint32_t)min((tensor_words - wg_words) * 4, (size_t)0xffffffffu), kBufferRsrcWord3);
    const uint32_t wlo = (uint32_t)(((g * TN + role * 2 + hsel) * 8 * K + j * K) * 4);
    const uint32_t wlo_prev = wlo + (uint32_t)(prev_off * 4);
    const uint32_t qbytes = (uint32_t)qstride * 4u, last_off = (uint32_t)qlast * qbytes;
    auto fetch_counted = [&](uint32_t(&w)[K + 1], int step) {
      buffer_slice_counted<K>(wrsrc, min((uint32_t)step * qbytes, last_off), wlo, wlo_prev, w);
    };
    uint32_t sl[PD][K + 1];
#pragma unroll
    for (int d = 0; d < PD; ++d)
      load_slice_prev<K>(tp + (size_t)min(d, qlast) * qstride, prev_off, sl[d]);
    // A: row 8i + (lane >> 3) of the consumer's 16*MB rows; the lane's slot is
    // lane & 7.  At MB >= 2 (trellis slices loaded with a known count of
    // instructions, buffer_slice_counted) A goes global -> LDS directly (lds_dma16_s: lane l
    // of a load fills bytes 16l..16l+15 of its 1 KB region, 8 rows; the swizzle
    // goes to the global side: slot s of row r reads chunk s ^ a_swizzle(r)),
    // issued when the stage frees and waited for before the iteration's barrier
    // with the slice issued after it still in flight (same-box A/B, 4096 ->
    // 14336: M=512 87.1 -> 84.7 us, M=256 57.7 -> 56.3, M=2048 324.6 -> 316);
    // MB = 1 (an iteration too short to cover the L2 latency of a copy issued at
    // its start: 45.9 -> 46.7 us at M=128) goes through registers two steps
    // ahead.
    constexpr bool kDma = MB >= 2;
    const int ar = lane >> 3, ac = lane & 7;
    const uint16_t* ap[2 * MB];
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i) {
      const int row = row_base + 8 * i + ar;
      ap[i] = mm.xhat + (size_t)(row < p.M ? row : 0) * p.in + (size_t)qa * 64 + ac * 8;
    }
    // direct copies: the row tile's first row and the step in the scalar
    // base, the lane's row (rows >= M read the tile's first row) and chunk in
    // a 32-bit byte offset
    const int tile_row0 = mtile * 64 * MB;
    const uint16_t* abase = mm.xhat + (size_t)tile_row0 * p.in + (size_t)qa * 64;
    uint32_t aoff[2 * MB];
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i) {
      const int r = role * 16 * MB + 8 * i + ar;  // row inside the tile
      aoff[i] = (uint32_t)(((tile_row0 + r < p.M ? r : 0) * p.in + (ac ^ a_swizzle(8 * i + ar)) * 8) * 2);
    }
    auto dma_a = [&](int step, int st) {
      const uint32_t base = __builtin_amdgcn_readfirstlane(
          lds_offset(astage(st) + role * (16 * MB * 128)));
      const uint16_t* sb = abase + (size_t)min(step, qlast) * 64;
#pragma unroll
      for (int i = 0; i < 2 * MB; ++i) lds_dma16_s(sb, aoff[i], base + i * 1024);
    };
    // A rows of steps q+2 and q+3 in flight (register sets alternate by step)
    u32x4 areg[2][kDma ? 1 : 2 * MB];
    auto load_a = [&](auto& dst, int step) {
#pragma unroll
      for (int i = 0; i < 2 * MB; ++i)
        dst[i] = *(const u32x4*)(ap[i] + (size_t)min(step, qlast) * 64);
    };
    auto store_a = [&](const auto& src, int st) {
      uint8_t* base = astage(st) + role * (16 * MB * 128);
#pragma unroll
      for (int i = 0; i < 2 * MB; ++i) {
        const int r = 8 * i + ar;
        *(u32x4*)(base + r * 128 + ((ac ^ a_swizzle(r)) << 4)) = src[i];
      }
    };
    // steps 0 and 1
    if constexpr (kDma) {
      dma_a(0, 0);
      dma_a(1, 1);
      __builtin_amdgcn_sched_barrier(0);
      qmm_produce<K, CB>(sl[0], bstage(0) + role * 256, lane);
      qmm_produce<K, CB>(sl[1], bstage(1) + role * 256, lane);
      __builtin_amdgcn_sched_barrier(0);
      fetch_counted(sl[0], PD);
      fetch_counted(sl[1], PD + 1);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * kSliceLoads<K>));
    } else {
      load_a(areg[0], 0);
      load_a(areg[1], 1);
      qmm_produce<K, CB>(sl[0], bstage(0) + role * 256, lane);
      load_slice_prev<K>(tp + (size_t)min(PD, qlast) * qstride, prev_off, sl[0]);
      qmm_produce<K, CB>(sl[1], bstage(1) + role * 256, lane);
      load_slice_prev<K>(tp + (size_t)min(PD + 1, qlast) * qstride, prev_off, sl[1]);
      store_a(areg[0], 0);
      load_a(areg[0], 2);
      store_a(areg[1], 1);
      load_a(areg[1], 3);
    }
    __syncthreads();
    // iteration q (slot (q+2) % 4 and A set q % 2 hold step q+2):
    // unconditional, so the load count per iteration is static (past-the-end
    // steps re-read the last one into a stage no consumer reads)
    auto iter = [&](int q, auto phase) {
      constexpr int P = decltype(phase)::value;
      const int st = (q + 2) % 3;
      if constexpr (kDma) {
        // stage st (step q-1) was released by the last barrier
        dma_a(q + 2, st);
        __builtin_amdgcn_sched_barrier(0);
        qmm_produce<K, CB>(sl[(P + 2) % PD], bstage(st) + role * 256, lane);
        __builtin_amdgcn_sched_barrier(0);
        fetch_counted(sl[(P + 2) % PD], q + 2 + PD);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kSliceLoads<K>));  // A of step q+2 has landed
      } else {
        qmm_produce<K, CB>(sl[(P + 2) % PD], bstage(st) + role * 256, lane);
        load_slice_prev<K>(tp + (size_t)min(q + 2 + PD, qlast) * qstride, prev_off,
                           sl[(P + 2) % PD]);
        store_a(areg[P & 1], st);
        load_a(areg[P & 1], q + 4);
      }
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
    if (p.splits > 1) {
      // split-K arrival: after every consumer's partials are acknowledged
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (uint32_t)(p.splits - 1);
        if (s_last)
          __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!s_last) return;  // uniform across the workgroup
    }
  } else {
    // ---- consumer `role`: 16*MB rows x 128 columns ----
    float4v acc[MB][8];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int f = 0; f < 8; ++f) acc[mb][f] = float4v{0.f, 0.f, 0.f, 0.f};
    // fragment (mb, h): row 16mb + n of this consumer, chunk 2g + h
    int aoff[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = role * 16 * MB + 16 * mb + n;
        aoff[mb][h] = r * 128 + (((2 * g + h) ^ a_swizzle(r)) << 4);
      }
    half8 a[2][MB][2], b[2][4];
    auto read_a = [&](half8(&dst)[MB][2], int st) {
      const uint8_t* base = astage(st);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int h = 0; h < 2; ++h) dst[mb][h] = *(const half8*)(base + aoff[mb][h]);
    };
    auto read_b = [&](half8(&dst)[4], int st, int w2) {
      const u32x4* bb = bstage(st) + w2 * 256 + lane;
#pragma unroll
      for (int f = 0; f < 4; ++f) dst[f] = __builtin_bit_cast(half8, bb[f * 64]);
    };
    __syncthreads();
    read_a(a[0], 0);
    read_b(b[0], 0, 0);
    // iteration q: A of step q in a[q&1], B groups alternate between b[0]
    // and b[1]; the last group prefetches step q+1 (stage (q+1) % 3)
    auto iter = [&](int q, auto phase) {
      constexpr int P = decltype(phase)::value;
      const int st = q % 3, st1 = (q + 1) % 3;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        if (w2 < 3) {
          read_b(b[(w2 + 1) & 1], st, w2 + 1);
        } else {
          read_a(a[(P + 1) & 1], st1);
          read_b(b[0], st1, 0);
        }
        // keep the reads of the next group ahead of this group's MFMAs
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int cg = 0; cg < 2; ++cg)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              acc[mb][w2 * 2 + cg] =
                  mfma16(a[P & 1][mb][h], b[w2 & 1][h * 2 + cg], acc[mb][w2 * 2 + cg]);
        __builtin_amdgcn_sched_barrier(0);
      }
      __syncthreads();
    };
    const int nq2 = nq & ~1;
    for (int q = 0; q < nq2; q += 2) {
      iter(q, std::integral_constant<int, 0>{});
      iter(q + 1, std::integral_constant<int, 1>{});
    }
    if (nq2 < nq) iter(nq2, std::integral_constant<int, 0>{});
    // the stages are free after the loop's last barrier
    auto stage_rows = [&]() {
      // static_for: the accumulator index must stay a compile-time constant
      static_for<MB>([&](auto mb_) {
        constexpr int mb = decltype(mb_)::value;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v[8];
#pragma unroll
          for (int f = 0; f < 8; ++f) v[f] = round_f16(acc[mb][f][r]);
          qmm_stage_row(v, lane, ys + (role * 16 * MB + 16 * mb + 4 * g + r) * kYStride);
        }
      });
    };
    if (p.splits == 1) {
      stage_rows();
    } else {
      // split-K: this part's accumulators out in fragment order (16 coalesced
      // bytes per lane and fragment) through agent-scope coherent stores (sc1)
      const __amdgpu_buffer_rsrc_t mine = qmm_slab(p, split, tile, MB);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int f = 0; f < 8; ++f)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mb][f]), mine,
                                                 ((role * MB + mb) * 8 + f) * 1024 + lane * 16, 0,
                                                 kCpolSc1);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();  // every part stored (the producers count the arrival)
      __syncthreads();
      if (!s_last) return;  // uniform across the workgroup
    }
  }
  if (p.splits > 1) {
    // the last part to arrive: every fragment summed over the parts in split
    // order (coherent 16-byte loads, all 8 waves, 4*MB fragments each, the
    // loads of kSumFrags fragments x kSumParts parts in flight together: one
    // round trip to the coherence point per group, not per load), its four
    // rows rounded to f16 into the tile's rows in LDS
    constexpr int kSumFrags = 4, kSumParts = 4;
    const int col = 16 * (n >> 3) + (n & 7);
    for (int i0 = 0; i0 < 4 * MB; i0 += kSumFrags) {
      float4v sum[kSumFrags];
#pragma unroll
      for (int i = 0; i < kSumFrags; ++i) sum[i] = float4v{0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < p.splits; s0 += kSumParts) {
        u32x4 t[kSumParts][kSumFrags];
#pragma unroll
        for (int c = 0; c < kSumParts; ++c) {
          // clamped: always a written part (the extra loads are not added)
          const __amdgpu_buffer_rsrc_t src = qmm_slab(p, min(s0 + c, p.splits - 1), tile, MB);
#pragma unroll
          for (int i = 0; i < kSumFrags; ++i)
            t[c][i] = __builtin_amdgcn_raw_buffer_load_b128(
                src, (wave * 4 * MB + i0 + i) * 1024 + lane * 16, 0, kCpolSc1);
        }
#pragma unroll
        for (int c = 0; c < kSumParts; ++c)
#pragma unroll
          for (int i = 0; i < kSumFrags; ++i)
            sum[i] = add_if(s0 + c < p.splits, sum[i], __builtin_bit_cast(float4v, t[c][i]));
      }
#pragma unroll
      for (int i = 0; i < kSumFrags; ++i) {
        const int slot = wave * 4 * MB + i0 + i;  // (consumer, mb, f)
        const int cr = slot / (8 * MB), mb = (slot / 8) % MB, f = slot % 8;
        uint16_t* y = ys + (cr * 16 * MB + 16 * mb + 4 * g) * kYStride + 32 * (f >> 1) +
                      8 * (f & 1) + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r * kYStride] = f2h(sum[i][r]);
      }
    }
  }
  __syncthreads();

  // ---- epilogue: all 8 waves finish 8*MB rows each, 4 rows per pass ----
  {
    const int colb = cblk_l * 128;
    const int chunk = lane & 15;
    float sv[8], bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sv[j] = s_svh[8 * chunk + j];
      bv[j] = s_bias[8 * chunk + j];
    }
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i) {
      const int rl = wave * 8 * MB + 4 * i + (lane >> 4);
      const int row = mtile * 64 * MB + rl;
      const u32x4 raw = *(const u32x4*)(ys + rl * kYStride + 8 * chunk);
      qmm_finish_chunk(raw, sv, bv, lane, row < p.M, mm, p.x_dtype,
                       (size_t)row * mm.out + colb + 8 * chunk);
    }
  }
}

}  // namespace exl3
