// MoE SwitchGLU over EXL3 expert banks: the reference's Exl3SwitchGlu
// (native/src/moe.rs:611-1085) -- route plan, routed inputs, expert QMMs,
// SwiGLU glue, down projection, weighted top-k reduction -- re-designed for
// gfx950 as four launches:
//   1. route:   workgroup 0 counting-sorts the rows*top_k slots by expert, cuts
//               each expert's run into blocks of <= 16, 32 or 64 rows (block
//               table) and clears the tile arrival counters of the two expert
//               QMMs; the other workgroups gather f16(x[token] * gu_suh[e][p])
//               -> staged Hadamard-128 for the gate (p = 0) and up (p = 1)
//               inputs, stored by slot;
//   2. gate/up: per (block, 128 hidden columns, K-range) a workgroup of 8 waves
//               decodes the expert's gate (waves 0-3) and up (waves 4-7) tiles of
//               those columns in registers -- each wave owns a column pair, as in
//               the QMV -- and multiplies them with the block's rows (read by
//               slot through the sorted order); the
//               epilogue is the whole of glu_down_input (moe.rs:435-563): f16,
//               f32 Hadamard, *scale*svh, SiLU(g)*u, *down_suh, f32 Hadamard,
//               *scale -> the down projection's xhat (GELU banks,
//               forward_gelu: staged Hadamards and GEGLU instead);
//   3. down:    the same kernel with 4 waves over the down bank; the epilogue is
//               finish_and_reduce's per-slot part (moe.rs:586-609): f16, staged
//               Hadamard, *svh, *score (f16 scores: an f16 product; f32 or bf16
//               scores: an f32 product, MLX's promotion), stored per slot;
//   4. reduce:  y[row] = sum over top_k in slot order in f32, then f16 (f16
//               scores) or kept f32 (f32 or bf16 scores).
// Small inputs (decode: a handful of slots) split K over several workgroups
// whose f32 partials meet in the last arriving one (agent-scope relaxed
// atomics, as in the QMV), which adds them in split order.  Each row's
// arithmetic is independent of the other rows of its block, so the
// (atomics-ordered) placement of slots inside an expert's run cannot change any
// result.
#pragma once

#include "exl3_device.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {

// Rows per block-table entry: up to 4 MFMA row blocks; the plan cuts 16-row
// blocks for small inputs (more workgroups) and 64-row blocks otherwise (each
// decoded weight serves more rows), as moe.rs:80-83 cuts 64.
constexpr int kMoeMaxBlockRows = 64;

struct MoePlanParams {
  const uint32_t* selected;  // [slots] expert ids (rows * top_k)
  int slots, experts;
  int* rank;                 // [slots] scratch
  int* sorted_slot;          // [slots] slot at each sorted position
  int4* table;               // [max_blocks] (expert, first sorted position, rows, 0)
  int* counts;               // [2]: block-table entries, routed slots
  int* expert_count;         // [experts] (rows routed to each expert)
  uint32_t* counters;        // [ncounters] tile arrival counters, cleared here
  int ncounters;
  int block_rows;            // 16, 32 or 64
};

// The route plan, run by one workgroup of NT threads: counting sort of the
// slots by expert, exclusive scans of the per-expert row and block counts,
// the block table.  Slots with an expert id >= experts are left out (their
// contribution is zero).  LDS (dynamic): cnt[E], off[E], boff[E+1].
template <int NT>
__device__ __forceinline__ void moe_plan_block(const MoePlanParams& p) {
  extern __shared__ int lds[];
  __shared__ int wsum[2][NT / 64];
  int* cnt = lds;
  int* off = lds + p.experts;
  int* boff = lds + 2 * p.experts;
  const int tid = threadIdx.x;
  for (int i = tid; i < p.ncounters; i += NT) p.counters[i] = 0u;
  for (int e = tid; e < p.experts; e += NT) cnt[e] = 0;
  __syncthreads();
  // each thread's expert ids are loaded kPlanBatch at a time (clamped: always
  // a valid slot), not one dependent round trip per slot
  constexpr int kPlanBatch = 8;
  for (int s0 = tid; s0 < p.slots; s0 += kPlanBatch * NT) {
    uint32_t e[kPlanBatch];
#pragma unroll
    for (int u = 0; u < kPlanBatch; ++u) e[u] = p.selected[min(s0 + u * NT, p.slots - 1)];
#pragma unroll
    for (int u = 0; u < kPlanBatch; ++u) {
      const int s = s0 + u * NT;
      if (s < p.slots) p.rank[s] = e[u] < (uint32_t)p.experts ? atomicAdd(&cnt[e[u]], 1) : -1;
    }
  }
  __syncthreads();
  // exclusive scans of the counts and block counts: each thread sums a run of
  // experts, the NT run totals are scanned (waves, then wave totals), and
  // each thread writes its run's offsets
  const int per = (p.experts + NT - 1) / NT;
  const int e0 = min(tid * per, p.experts), e1 = min(e0 + per, p.experts);
  int lc = 0, lb = 0;
  for (int e = e0; e < e1; ++e) {
    lc += cnt[e];
    lb += (cnt[e] + p.block_rows - 1) / p.block_rows;
  }
  int ic = lc, ib = lb;  // inclusive scan inside the wave
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int tc = __shfl_up(ic, d, 64), tb = __shfl_up(ib, d, 64);
    if (lane >= d) ic += tc, ib += tb;
  }
  if (lane == 63) wsum[0][wv] = ic, wsum[1][wv] = ib;
  __syncthreads();
  int bc = 0, bb = 0;
  for (int w = 0; w < wv; ++w) bc += wsum[0][w], bb += wsum[1][w];
  int rc = bc + ic - lc, rb = bb + ib - lb;  // exclusive prefix of this run
  for (int e = e0; e < e1; ++e) {
    off[e] = rc;
    boff[e] = rb;
    rc += cnt[e];
    rb += (cnt[e] + p.block_rows - 1) / p.block_rows;
  }
  if (tid == NT - 1) {
    boff[p.experts] = rb;
    p.counts[0] = rb;
    p.counts[1] = rc;
  }
  __syncthreads();
  for (int s0 = tid; s0 < p.slots; s0 += kPlanBatch * NT) {
    int r[kPlanBatch];
    uint32_t e[kPlanBatch];
#pragma unroll
    for (int u = 0; u < kPlanBatch; ++u) {
      const int s = min(s0 + u * NT, p.slots - 1);
      r[u] = p.rank[s];
      e[u] = p.selected[s];
    }
#pragma unroll
    for (int u = 0; u < kPlanBatch; ++u) {
      const int s = s0 + u * NT;
      if (s < p.slots && r[u] >= 0) p.sorted_slot[off[e[u]] + r[u]] = s;
    }
  }
  for (int e = tid; e < p.experts; e += NT) {
    p.expert_count[e] = cnt[e];
    for (int b = boff[e]; b < boff[e + 1]; ++b) {
      const int first = off[e] + (b - boff[e]) * p.block_rows;
      p.table[b] = make_int4(e, first, min(p.block_rows, off[e] + cnt[e] - first), 0);
    }
  }
}

struct MoeGatherParams {
  const void* x;              // [rows][in] activations (f16, bf16 or f32)
  int x_dtype, in, top_k, slots, experts;
  const uint32_t* selected;   // [slots]
  const uint16_t* gu_suh;     // [E][2][in]
  uint16_t* xgu;              // [2][slots][in]
};

// Gate/up inputs in slot order: xgu[proj][slot][in] = f16(x[slot / top_k] *
// gu_suh[e][proj]) -> staged Hadamard-128 (routed_inputs, moe.rs:184-250),
// proj 0 = gate, 1 = up.  One wave per (slot, projection, run of 8
// 128-blocks), 16 lanes per block (prologue8), each lane's two blocks loaded
// together.  The activation loads need no routing data, so they go out before
// the expert id arrives; slots routed to no valid expert are computed from
// expert 0's scales and not stored (no block reads them).
template <bool VEC>
__device__ __forceinline__ void moe_gather_wave(const MoeGatherParams& p, int job, int lane) {
  const int nb = p.in >> 7, runs = (nb + 7) >> 3;
  const int pp = job / runs, run = job - pp * runs;
  const int slot = pp >> 1, proj = pp & 1;
  if (slot >= p.slots) return;  // uniform per wave
  const size_t xrow = (size_t)(slot / p.top_k) * p.in;
  const int b0 = 8 * run + (lane >> 4), b1 = b0 + 4;
  const int bl = min(b1, nb - 1);  // clamped: the second block's lanes stay in bounds
  const int c0 = b0 * 128 + 8 * (lane & 15), c1 = bl * 128 + 8 * (lane & 15);
  // a group past the row's end (its last run holding fewer than 4 blocks)
  // recomputes block nb - 1 without storing
  const int c0c = b0 < nb ? c0 : (nb - 1) * 128 + 8 * (lane & 15);
  if constexpr (VEC) {
    if (p.x_dtype == DT_F16) {  // packed f16 products (scale8_f16)
      const uint16_t* xh = (const uint16_t*)p.x + xrow;
      const u32x4 x0 = *(const u32x4*)(xh + c0c), x1 = *(const u32x4*)(xh + c1);
      const uint32_t e = p.selected[slot];
      const bool live = e < (uint32_t)p.experts;
      const uint16_t* suh = p.gu_suh + ((size_t)(live ? e : 0u) * 2 + proj) * p.in;
      float v0[8], v1[8];
      scale8_f16(x0, *(const u32x4*)(suh + c0c), v0);
      scale8_f16(x1, *(const u32x4*)(suh + c1), v1);
      uint16_t* dst = p.xgu + ((size_t)proj * p.slots + slot) * p.in;
      finish8_scaled<VEC>(v0, dst + c0c, live && b0 < nb, lane);
      finish8_scaled<VEC>(v1, dst + c1, live && b1 < nb, lane);
      return;
    }
  }
  float a0[8], s0[8], a1[8], s1[8];
  load8_act<VEC>(p.x, p.x_dtype, xrow + c0c, a0);
  load8_act<VEC>(p.x, p.x_dtype, xrow + c1, a1);
  const uint32_t e = p.selected[slot];
  const bool live = e < (uint32_t)p.experts;
  const uint16_t* suh = p.gu_suh + ((size_t)(live ? e : 0u) * 2 + proj) * p.in;
  load8_scale<VEC>(suh + c0c, s0);
  load8_scale<VEC>(suh + c1, s1);
  uint16_t* dst = p.xgu + ((size_t)proj * p.slots + slot) * p.in;
  finish8<VEC>(a0, s0, dst + c0c, live && b0 < nb, lane);
  finish8<VEC>(a1, s1, dst + c1, live && b1 < nb, lane);
}

// Launch 1 of the forward: workgroup 0 builds the route plan while the
// others gather the gate/up inputs, which are stored by slot and so need
// nothing from the plan.  grid 1 + ceil(2 * slots * ceil(in / 1024) / 4),
// 256 threads, (3 * experts + 1) ints of dynamic LDS.
template <bool VEC>
__global__ __launch_bounds__(256) void moe_route_kernel(MoePlanParams pp, MoeGatherParams gp) {
  if (blockIdx.x == 0) {
    moe_plan_block<256>(pp);
    return;
  }
  const int job = __builtin_amdgcn_readfirstlane((blockIdx.x - 1) * 4 + (threadIdx.x >> 6));
  moe_gather_wave<VEC>(gp, job, threadIdx.x & 63);
}

struct MoeMmParams {
  const uint32_t* trellis;  // bank, [k_in/16][tn_total][8K] u32
  int tn_total;             // tile columns of the bank
  int k_in;                 // input width of the projection (rows of the trellis)
  int width;                // output width of one expert's projection
  int experts;
  const int4* table;
  const int* counts;        // [0] = block-table entries
  const int* sorted_slot;
  int col_blocks;           // width / 128
  int splits;               // K-ranges per (block, column block)
  int slots_pad;            // position stride of xa / partials
  const uint16_t* xa;       // A rows [nproj][slots_pad][k_in] (f16, rotated)
  const int* a_rows;        // A row of each sorted position (gate/up: its slot,
                            // as the route launch stores them); null: the position
  float* partials;          // [splits][nproj][slots_pad][width] (splits > 1)
  uint32_t* counters;       // [blocks][col_blocks], cleared by the plan
  // gate/up epilogue
  const uint16_t* gu_svh;   // [E][2][width]
  const uint16_t* down_suh; // [E][width]
  uint16_t* xd;             // [slots_pad][width]
  int gelu;                 // 0: SiLU (glu_down_input), 1: GELU (forward_gelu)
  int logical_hidden;       // GELU: outputs of columns >= logical_hidden are zero
  // down epilogue
  const uint16_t* down_svh; // [E][width]
  const void* scores;       // [slots] of scores_dtype
  int scores_dtype;         // f16: f16 products; f32 / bf16: f32 products
  void* z;                  // [slots][width], f16 (f16 scores) or f32
};

// A routing score as f32 (f16, bf16 or f32 storage).
__device__ __forceinline__ float load_score(const void* scores, int dt, size_t i) {
  if (dt == DT_F32) return ((const float*)scores)[i];
  const uint16_t b = ((const uint16_t*)scores)[i];
  return dt == DT_BF16 ? bf2f(b) : h2f(b);
}

// One slot's weighted output value (finish_and_reduce, moe.rs:604-607): the
// f16 value times its score -- rounded to f16 when the score is f16, an f32
// product otherwise (MLX promotes f16 * f32 and f16 * bf16 to f32).
__device__ __forceinline__ float weighted(float v16, float score, int scores_dtype) {
  return scores_dtype == DT_F16 ? round_f16(v16 * score) : v16 * score;
}

// finish_and_reduce's per-slot part (moe.rs:586-609) for columns (lane,
// lane + 64) of a 128-column block of the down projection's f32 sums (g0, g1):
// f16(raw) -> staged Hadamard -> f16(* scale) -> f16(* svh) -> * score
// (weighted).
__device__ __forceinline__ void moe_down_values(const MoeMmParams& p, int e, int slot, int cblk,
                                                float g0, float g1, int lane, float& v0,
                                                float& v1) {
  v0 = round_f16(g0);
  v1 = round_f16(g1);
  h128_wave<true>(v0, v1, lane);
  v0 = round_f16(v0 * kHadScale);
  v1 = round_f16(v1 * kHadScale);
  const uint16_t* sv = p.down_svh + (size_t)e * p.width + cblk * 128;
  const float sc = load_score(p.scores, p.scores_dtype, slot);
  v0 = weighted(round_f16(v0 * h2f(sv[lane])), sc, p.scores_dtype);
  v1 = weighted(round_f16(v1 * h2f(sv[lane + 64])), sc, p.scores_dtype);
}

// Stores one reduced output value: f16 for f16 scores, f32 otherwise (the
// dtype MLX's promotion gives the weighted sum).
__device__ __forceinline__ void store_reduced(void* y, int scores_dtype, size_t i, float v) {
  if (scores_dtype == DT_F16)
    ((uint16_t*)y)[i] = f2h(v);
  else
    ((float*)y)[i] = v;
}

// The token `row`'s output columns (lane, lane + 64) of 128-column block
// `cblk`: the sum over its valid slots in top-k order of their weighted values
// (f32 z rows, f32 adds, as moe_reduce_kernel), stored as f16 or f32; the
// slots' ids and values load kTopChunk slots at a time (rows of slots outside
// the bank are loaded, never added).
__device__ __forceinline__ void moe_token_sum(const MoeMmParams& p, const uint32_t* selected,
                                              int top_k,
                                              const float* zf, void* y, int row, int cblk,
                                              int lane) {
  constexpr int kTopChunk = 8;
  float y0 = 0.f, y1 = 0.f;
  for (int t0 = 0; t0 < top_k; t0 += kTopChunk) {
    uint32_t ids[kTopChunk];
    float a[kTopChunk], b[kTopChunk];
#pragma unroll
    for (int c = 0; c < kTopChunk; ++c) {
      const size_t ts = (size_t)row * top_k + min(t0 + c, top_k - 1);
      ids[c] = selected[ts];
      const float* zr = zf + ts * p.width + cblk * 128;
      a[c] = load_coherent(zr + lane);
      b[c] = load_coherent(zr + lane + 64);
    }
#pragma unroll
    for (int c = 0; c < kTopChunk; ++c) {
      const bool live = t0 + c < top_k && ids[c] < (uint32_t)p.experts;
      y0 = add_if(live, y0, a[c]);
      y1 = add_if(live, y1, b[c]);
    }
  }
  const size_t o = (size_t)row * p.width + cblk * 128 + lane;
  store_reduced(y, p.scores_dtype, o, y0);
  store_reduced(y, p.scores_dtype, o + 64, y1);
}

// Epilogue of one routed row of a 128-column block: (g0, g1) and (u0, u1) are
// the f32 sums of columns (lane, lane+64) of the first and last projection.
template <bool GLU>
__device__ __forceinline__ void moe_finish_row(const MoeMmParams& p, int e, int pos, int cblk,
                                               float g0, float g1, float u0, float u1,
                                               int lane) {
  const int col0 = cblk * 128;
  if constexpr (GLU) {
    const uint16_t* gsv = p.gu_svh + ((size_t)e * 2) * p.width + col0;
    const uint16_t* usv = gsv + p.width;
    const uint16_t* dsu = p.down_suh + (size_t)e * p.width + col0;
    uint16_t* dst = p.xd + (size_t)pos * p.width + col0;
    g0 = round_f16(g0), g1 = round_f16(g1), u0 = round_f16(u0), u1 = round_f16(u1);
    if (p.gelu) {  // uniform
      // forward_gelu (moe.rs:1087-1153): gate and up as expert_mapped returns
      // them (linear.rs:3325-3331: f16, staged Hadamard, f16(* scale),
      // f16(* svh)), GEGLU with zeros from logical_hidden on, then the down
      // input as expert_mapped prepares it (linear.rs:3131-3137: f16(h *
      // down_suh), staged Hadamard, f16(* scale))
      h128_wave<true>(g0, g1, lane);
      h128_wave<true>(u0, u1, lane);
      g0 = round_f16(round_f16(g0 * kHadScale) * h2f(gsv[lane]));
      g1 = round_f16(round_f16(g1 * kHadScale) * h2f(gsv[lane + 64]));
      u0 = round_f16(round_f16(u0 * kHadScale) * h2f(usv[lane]));
      u1 = round_f16(round_f16(u1 * kHadScale) * h2f(usv[lane + 64]));
      const float a0 = col0 + lane < p.logical_hidden ? geglu_f16(g0, u0) : 0.f;
      const float a1 = col0 + lane + 64 < p.logical_hidden ? geglu_f16(g1, u1) : 0.f;
      float d0 = round_f16(a0 * h2f(dsu[lane])), d1 = round_f16(a1 * h2f(dsu[lane + 64]));
      h128_wave<true>(d0, d1, lane);
      dst[lane] = f2h(d0 * kHadScale);
      dst[lane + 64] = f2h(d1 * kHadScale);
      return;
    }
    // gate and up: f16(raw) -> f32 Hadamard -> f16(v * scale * svh)
    h128_wave<false>(g0, g1, lane);
    h128_wave<false>(u0, u1, lane);
    g0 = round_f16(g0 * kHadScale * h2f(gsv[lane]));
    g1 = round_f16(g1 * kHadScale * h2f(gsv[lane + 64]));
    u0 = round_f16(u0 * kHadScale * h2f(usv[lane]));
    u1 = round_f16(u1 * kHadScale * h2f(usv[lane + 64]));
    // SiLU(g) * u, then * down_suh, f32 Hadamard, f16(v * scale)
    const float a0 = round_f16((g0 / (1.0f + expf(-g0))) * u0);
    const float a1 = round_f16((g1 / (1.0f + expf(-g1))) * u1);
    float d0 = round_f16(a0 * h2f(dsu[lane])), d1 = round_f16(a1 * h2f(dsu[lane + 64]));
    h128_wave<false>(d0, d1, lane);
    dst[lane] = f2h(d0 * kHadScale);
    dst[lane + 64] = f2h(d1 * kHadScale);
  } else {
    (void)u0, (void)u1;
    const int slot = p.sorted_slot[pos];
    float v0, v1;
    moe_down_values(p, e, slot, cblk, g0, g1, lane, v0, v1);
    const size_t at = (size_t)slot * p.width + col0 + lane;
    if (p.scores_dtype == DT_F16) {
      ((uint16_t*)p.z)[at] = f2h(v0);
      ((uint16_t*)p.z)[at + 64] = f2h(v1);
    } else {
      ((float*)p.z)[at] = v0;
      ((float*)p.z)[at + 64] = v1;
    }
  }
}

// Grouped expert QMM over one block of up to 16*MB rows, one 128-column block
// and one K-range.  NPROJ = 2 (gate/up, GLU epilogue) or 1 (down).  Wave w
// serves projection w / 4 and the column pair w % 4 with the QMV's loop: D
// trellis slices in flight per set, two sets in ping-pong, unconditional
// (clamped) loads.  Each decoded step feeds the block's ceil(rows/16) row
// groups.  The register budget asks for 4 waves per SIMD (two gate/up
// workgroups per CU) where that needs no spill; the MUL1 decode (CB = 2) and the
// 64-row blocks get 3 and 2.
template <int K, int CB, int NPROJ, int MB>
__global__ __launch_bounds__(256 * NPROJ)
__attribute__((amdgpu_waves_per_eu(MB == 4 ? 2 : CB == 2 ? 3 : 4))) void moe_mm_kernel(
    MoeMmParams p) {
  // A rows of the block pass through LDS in chunks of C = D steps, two chunks
  // deep: [buffer][step][proj][row][8 chunks of 16 bytes], chunk c of row r at
  // slot c ^ a_swizzle(r) so that the 16-row fragment reads are conflict-free.
  // The rows go global -> LDS directly (global_load_lds_dwordx4: lane l of a
  // load fills bytes 16l..16l+15 of its 1 KB region, 8 rows of one
  // projection, the swizzle applied to the global address), one barrier per
  // chunk.  After the loop the same bytes hold the row-group sums.
  // trellis slices per set and steps per A chunk: 2 (same box, C4: 147.0 ->
  // 144.2 us against the 4 of the weight-stream default at K <= 4)
  constexpr int D = 2, C = D;
  constexpr int kRows = 16 * MB, kStep = NPROJ * kRows * 128, kBuf = C * kStep;
  constexpr int kRed = NPROJ * 16 * 128 * 4;
  // two separate objects, so that the compiler sees the loads into one buffer
  // cannot alias the fragment reads of the other (no wait before those reads)
  __shared__ __attribute__((aligned(16))) uint8_t abuf0[kBuf > kRed ? kBuf : kRed];
  __shared__ __attribute__((aligned(16))) uint8_t abuf1[kBuf];
  float(*red)[16][128] = (float(*)[16][128])abuf0;  // f32 sums of one row group (one K-range)
  __shared__ int s_last;
  constexpr bool GLU = NPROJ == 2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int proj = wave >> 2, pair = wave & 3;
  // Workgroup -> (block, column block, split).  Workgroups go to the 8 XCDs
  // round-robin (XCD = id % 8); XCD x takes blocks x, x + 8, x + 16, ...
  // whole, every column block and split of one, so the block's routed rows
  // are read from HBM once into that XCD's L2 instead of once per column
  // block.  The grid holds ceil(max_blocks / 8) * 8 blocks.
  const int per_blk = p.col_blocks * p.splits;
  const int wk = blockIdx.x >> 3;
  const int blk = (wk / per_blk) * 8 + (blockIdx.x & 7);
  const int wi = wk % per_blk;
  const int split = wi % p.splits, cblk = wi / p.splits;
  if (blk >= p.counts[0]) return;  // uniform
  const int4 ent = p.table[blk];
  const int e = ent.x, pos0 = ent.y, nrows = ent.z;
  const int groups = (nrows + 15) >> 4;
  const int nq_all = p.k_in >> 6;
  const int qa = split * nq_all / p.splits, nq = (split + 1) * nq_all / p.splits - qa;

  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7, am = lane & 15;
  const int tpe = p.width / 16;  // tile columns per expert
  const size_t qstride = (size_t)4 * p.tn_total * 8 * K;
  const int tcol = (proj * p.experts + e) * tpe + cblk * 8 + 2 * pair + hsel;
  const uint32_t* tp =
      p.trellis + ((size_t)(4 * qa + g) * p.tn_total + tcol) * (8 * K) + (size_t)j * K;
  const int prev_off = j == 0 ? 8 * K - 1 : -1;
  // A loads: a step is NI = NPROJ * kRows / 8 loads of 8 rows, load i covering
  // projection i / (kRows / 8) and rows 8 * (i % (kRows / 8)) + 0..7; wave w
  // issues loads w, w + 4 * NPROJ, ...  A load whose rows lie past the
  // block's row groups is skipped; rows past the block's end inside its last
  // group repeat its last row (their sums are never used).
  constexpr int NW = 4 * NPROJ, NI = NPROJ * kRows / 8, kPerW = (NI + NW - 1) / NW;
  const uint16_t* asrc[kPerW];
  int adst[kPerW];
  bool aact[kPerW];
#pragma unroll
  for (int i = 0; i < kPerW; ++i) {
    const int li = wave + i * NW;
    const int pj = li / (kRows / 8), row = 8 * (li % (kRows / 8)) + (lane >> 3);
    aact[i] = li < NI && (8 * (li % (kRows / 8))) / 16 < groups;  // uniform per wave
    const int at = pos0 + min(row, nrows - 1);
    const int arow = p.a_rows ? p.a_rows[at] : at;
    asrc[i] = p.xa + ((size_t)(li < NI ? pj : 0) * p.slots_pad + arow) * p.k_in +
              (size_t)qa * 64 + (((lane & 7) ^ a_swizzle(row)) << 3);
    adst[i] = (pj * kRows + 8 * (li % (kRows / 8))) * 128;
  }
  const int qlast = nq - 1;
  // chunk ch of A into buffer b (steps past the range re-read the last one
  // into slots no one reads, so every wave issues the same loads per chunk)
  auto load_chunk = [&](int ch, int b) {
#pragma unroll
    for (int d = 0; d < C; ++d) {
      const size_t qoff = (size_t)min(ch * C + d, qlast) * 64;
#pragma unroll
      for (int i = 0; i < kPerW; ++i)
        if (aact[i])
          __builtin_amdgcn_global_load_lds(
              (const void*)(asrc[i] + qoff),
              (__attribute__((address_space(3))) void*)((b ? abuf1 : abuf0) + d * kStep + adst[i]),
              16, 0, 0);
    }
  };
  // fragment (mb, h) of this lane: row 16mb + am of the wave's projection, chunk 2g + h
  int aoff[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 16 * mb + am;
      aoff[mb][h] = (proj * kRows + row) * 128 + (((2 * g + h) ^ a_swizzle(row)) << 4);
    }

  uint32_t setA[D][K + 1], setB[D][K + 1];
  auto fetch = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      load_slice_prev<K>(tp + (size_t)min(qbase + d, qlast) * qstride, prev_off, set[d]);
  };
  float4v acc0[MB], acc1[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc0[mb] = acc1[mb] = float4v{0.f, 0.f, 0.f, 0.f};
  // chunk ch (buffer ch & 1, trellis set `cur`): chunk ch + 1's A and trellis
  // go out first, into the other buffer and set; then its C steps are
  // multiplied; the wait and barrier at its end publish chunk ch + 1 and free
  // buffer ch & 1 for chunk ch + 2
  const int nch = (nq + C - 1) / C;
  auto chunk = [&](uint32_t(&cur)[D][K + 1], uint32_t(&nxt)[D][K + 1], int ch, int b) {
    if (ch + 1 < nch) load_chunk(ch + 1, b ^ 1);  // uniform
    fetch(nxt, (ch + 1) * C);
#pragma unroll
    for (int d = 0; d < C; ++d) {
      const int q = ch * C + d;
      if (q < nq) {  // uniform
        uint32_t src[32];
        extract_states<K>(cur[d], src);
        half8 b00 = decode_fragment<CB, K, 0, 0>(src);
        half8 b01 = decode_fragment<CB, K, 0, 1>(src);
        half8 b10 = decode_fragment<CB, K, 1, 0>(src);
        half8 b11 = decode_fragment<CB, K, 1, 1>(src);
        mfma_operand_fence(b00, b01);
        mfma_operand_fence(b10, b11);
        const uint8_t* st = (b ? abuf1 : abuf0) + d * kStep;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          if (mb < groups) {
            const half8 a0 = *(const half8*)(st + aoff[mb][0]);
            const half8 a1 = *(const half8*)(st + aoff[mb][1]);
            acc0[mb] = mfma16(a0, b00, acc0[mb]);
            acc1[mb] = mfma16(a0, b01, acc1[mb]);
            acc0[mb] = mfma16(a1, b10, acc0[mb]);
            acc1[mb] = mfma16(a1, b11, acc1[mb]);
          }
      }
      // steps stay in order (no decode hoisted across steps: register pressure)
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk ch + 1 have landed
    __syncthreads();
  };
  load_chunk(0, 0);
  fetch(setA, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int ch = 0; ch < nch; ch += 2) {
    chunk(setA, setB, ch, 0);
    if (ch + 1 < nch) chunk(setB, setA, ch + 1, 1);  // uniform
  }

  // accumulator lane l: rows 4*(l/16)+r, column 32*pair + 16*(n/8) + n%8 + 8*cg
  const int n = lane & 15;
  const int col = 32 * pair + 16 * (n >> 3) + (n & 7);
  if (p.splits == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if (mb >= groups) break;  // uniform
      if (mb > 0) __syncthreads();  // the previous group's rows are read
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[proj][4 * g + r][col] = acc0[mb][r];
        red[proj][4 * g + r][col + 8] = acc1[mb][r];
      }
      __syncthreads();
      const int rows = min(16, nrows - 16 * mb);
      for (int m = wave; m < rows; m += 4 * NPROJ)
        moe_finish_row<GLU>(p, e, pos0 + 16 * mb + m, cblk, red[0][m][lane],
                            red[0][m][lane + 64], red[NPROJ - 1][m][lane],
                            red[NPROJ - 1][m][lane + 64], lane);
    }
    return;
  }

  // split-K: partials out, count arrivals, the last arriver adds them up
  float* part = p.partials + ((size_t)split * NPROJ + proj) * p.slots_pad * p.width;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mb + 4 * g + r;
      if (m < nrows) {
        float* dst = part + (size_t)(pos0 + m) * p.width + cblk * 128 + col;
        store_coherent(dst, acc0[mb][r]);
        store_coherent(dst + 8, acc1[mb][r]);
      }
    }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t* counter = p.counters + (size_t)blk * p.col_blocks + cblk;
  if (threadIdx.x == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == (uint32_t)(p.splits - 1);
  }
  __syncthreads();
  if (!s_last) return;  // uniform
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // split sums in split order; the loads of kSplitChunk / NPROJ splits go out
  // together
  constexpr int kChunk = kSplitChunk / NPROJ;
  for (int m = wave; m < nrows; m += 4 * NPROJ) {
    float v[NPROJ][2] = {};
    for (int s0 = 0; s0 < p.splits; s0 += kChunk) {
      float t[kChunk][NPROJ][2];
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int s = min(s0 + c, p.splits - 1);  // clamped: always a written split
#pragma unroll
        for (int pj = 0; pj < NPROJ; ++pj) {
          const float* src = p.partials +
                             ((size_t)(s * NPROJ + pj) * p.slots_pad + pos0 + m) * p.width +
                             cblk * 128;
          t[c][pj][0] = load_coherent(src + lane);
          t[c][pj][1] = load_coherent(src + lane + 64);
        }
      }
#pragma unroll
      for (int c = 0; c < kChunk; ++c)
#pragma unroll
        for (int pj = 0; pj < NPROJ; ++pj) {
          v[pj][0] = add_if(s0 + c < p.splits, v[pj][0], t[c][pj][0]);
          v[pj][1] = add_if(s0 + c < p.splits, v[pj][1], t[c][pj][1]);
        }
    }
    moe_finish_row<GLU>(p, e, pos0 + m, cblk, v[0][0], v[0][1], v[NPROJ - 1][0],
                        v[NPROJ - 1][1], lane);
  }
}

// swiglu_down_input (moe.rs:569-583) as an op: the SiLU glue of
// moe_finish_row on f32 gate/up rows [2s], [2s+1] of slot s.  One wave per
// (slot, 128-column block); grid (slots, hidden / 128).  Slots routed to an
// expert id >= experts get zeros (the reference reads out of its bank).
__global__ __launch_bounds__(64) void swiglu_down_input_kernel(MoeMmParams p,
                                                               const float* __restrict__ gate_up,
                                                               const uint32_t* selected) {
  const int slot = blockIdx.x, cblk = blockIdx.y, lane = threadIdx.x;
  const uint32_t e = selected[slot];
  const size_t off = (size_t)2 * slot * p.width + cblk * 128;
  if (e >= (uint32_t)p.experts) {
    p.xd[(size_t)slot * p.width + cblk * 128 + lane] = 0;
    p.xd[(size_t)slot * p.width + cblk * 128 + lane + 64] = 0;
    return;
  }
  moe_finish_row<true>(p, (int)e, slot, cblk, gate_up[off + lane], gate_up[off + lane + 64],
                       gate_up[off + p.width + lane], gate_up[off + p.width + lane + 64], lane);
}

// finish_and_reduce (moe.rs:586-609) as an op: y[row] = sum_t of
// weighted(f16(H(f16(raw)) * svh), score) over slots row*top_k + t in t order
// (f32 adds), rounded to f16 for f16 scores; H the staged Hadamard with
// f16(v * scale), svh one row per slot.  One wave per (row, 128-column block);
// grid (rows, width / 128).
__global__ __launch_bounds__(64) void finish_and_reduce_kernel(const float* __restrict__ raw,
                                                               const uint16_t* __restrict__ svh,
                                                               const void* __restrict__ scores,
                                                               int scores_dtype, int top_k,
                                                               int width, void* __restrict__ y) {
  const int row = blockIdx.x, col = blockIdx.y * 128 + threadIdx.x, lane = threadIdx.x;
  float a0 = 0.f, a1 = 0.f;
  for (int t = 0; t < top_k; ++t) {
    const size_t slot = (size_t)row * top_k + t;
    float v0 = round_f16(raw[slot * width + col]), v1 = round_f16(raw[slot * width + col + 64]);
    h128_wave<true>(v0, v1, lane);
    const float sc = load_score(scores, scores_dtype, slot);
    a0 += weighted(round_f16(round_f16(v0 * kHadScale) * h2f(svh[slot * width + col])), sc,
                   scores_dtype);
    a1 += weighted(round_f16(round_f16(v1 * kHadScale) * h2f(svh[slot * width + col + 64])), sc,
                   scores_dtype);
  }
  store_reduced(y, scores_dtype, (size_t)row * width + col, a0);
  store_reduced(y, scores_dtype, (size_t)row * width + col + 64, a1);
}

// y[row][i] = sum_t z[row*top_k + t][i] in t order with f32 adds (z f16 for
// f16 scores, f32 otherwise), stored as f16 or f32 the same way; slots routed
// to no valid expert contribute zero.  Each thread owns 8 consecutive columns
// and issues the loads of 8 slots together (those of invalid slots, in bounds
// of z, are dropped), so a row costs one load latency per 8 slots.  VEC: y is
// 16-byte aligned.  grid (rows, ceil(width / 2048)), 256 threads.
template <bool VEC>
__global__ __launch_bounds__(256) void moe_reduce_kernel(const void* __restrict__ z,
                                                         int scores_dtype,
                                                         const uint32_t* __restrict__ selected,
                                                         int experts, int top_k, int width,
                                                         void* __restrict__ y) {
  const int i = (blockIdx.y * 256 + threadIdx.x) * 8, row = blockIdx.x;
  if (i >= width) return;
  const bool f16 = scores_dtype == DT_F16;
  float acc[8] = {};
  for (int t0 = 0; t0 < top_k; t0 += 8) {
    float v[8][8];
    bool ok[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int t = min(t0 + c, top_k - 1);
      const size_t slot = (size_t)row * top_k + t;
      ok[c] = t0 + c < top_k && selected[slot] < (uint32_t)experts;
      const size_t at = slot * width + i;
      if (f16) {
        const u32x4 w = *(const u32x4*)((const uint16_t*)z + at);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[c][2 * k] = h2f((uint16_t)w[k]);
          v[c][2 * k + 1] = h2f((uint16_t)(w[k] >> 16));
        }
      } else {
        const float4v w0 = *(const float4v*)((const float*)z + at);
        const float4v w1 = *(const float4v*)((const float*)z + at + 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[c][k] = w0[k], v[c][k + 4] = w1[k];
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] = add_if(ok[c], acc[k], v[c][k]);
  }
  const size_t o = (size_t)row * width + i;
  if (!VEC) {
#pragma unroll
    for (int k = 0; k < 8; ++k) store_reduced(y, scores_dtype, o + k, acc[k]);
  } else if (f16) {
    u32x4 w;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = (uint32_t)f2h(acc[2 * k]) | ((uint32_t)f2h(acc[2 * k + 1]) << 16);
    *(u32x4*)((uint16_t*)y + o) = w;
  } else {
    *(float4v*)((float*)y + o) = float4v{acc[0], acc[1], acc[2], acc[3]};
    *(float4v*)((float*)y + o + 4) = float4v{acc[4], acc[5], acc[6], acc[7]};
  }
}

// ---------------------------------------------------------------------------
// Small-row path (decode): one slot per workgroup row
// ---------------------------------------------------------------------------
// For a handful of routed slots (the reference runs rows < 64 through its
// small-row path, moe.rs:925-970) the forward is two launches with no route
// plan and no gather:
//   moe_dec_gu_kernel: per (slot, 128 hidden columns, K-range) a workgroup of
//     8 waves computes the slot's gate and up inputs for its K-range (the
//     gather's prologue8 on x and gu_suh[e]) into LDS, decodes expert e's gate
//     (waves 0-3) and up (waves 4-7) tiles and multiplies them with that one
//     row; the K-ranges meet in the last arriving workgroup, which runs
//     glu_down_input and writes the down projection's xhat of the slot;
//   moe_dec_down_kernel: per (slot, 128 output columns, K-range) 4 waves over
//     the down bank with the slot's xhat read from L2; the last arriver of the
//     K-ranges computes the slot's weighted values (finish_and_reduce's
//     per-slot part), and the last of a token's valid slots to finish a
//     column block sums them in top-k order into y.
// The K-ranges, the MFMA order of every step and the epilogues are those of
// moe_mm_kernel, so with the same split count every output equals the grouped
// path's bit for bit.  Arrival counters sit in the workspace's counter region
// (zero between calls, reset by each last arriver).  Slots routed to an
// expert id >= experts contribute nothing.
struct MoeDecParams {
  MoeMmParams m;             // bank, widths, epilogue scales, scores
  const void* x;             // [rows][in] activations
  int x_dtype, top_k, in;
  const uint32_t* selected;  // [slots]
  const uint16_t* gu_suh;    // [E][2][in]
  uint32_t* counters;        // gate/up: [slots][hidden/128]; down: [slots][in/128]
                             // then the top-k sums' [rows][in/128]
  float* zf;                 // [slots][in] weighted slot outputs (f32)
  void* y;                   // [rows][in] f16 (f16 scores) or f32
};

// Gate/up: grid slots * (hidden / 128) * splits, 512 threads.
template <int K, int CB>
__global__ __launch_bounds__(512) void moe_dec_gu_kernel(MoeDecParams dp) {
  const MoeMmParams& p = dp.m;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][16 * 128];  // xhat of the K-range
  __shared__ float red[2][128];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int proj = wave >> 2, pair = wave & 3;
  const int per_slot = p.col_blocks * p.splits;
  const int slot = blockIdx.x / per_slot, rem = blockIdx.x - slot * per_slot;
  const int cblk = rem / p.splits, split = rem - cblk * p.splits;
  const uint32_t eu = dp.selected[slot];
  if (eu >= (uint32_t)p.experts) return;  // uniform: a slot outside the bank adds nothing
  const int e = (int)eu, row = slot / dp.top_k;
  const int nq_all = p.k_in >> 6;
  const int qa = split * nq_all / p.splits, nq = (split + 1) * nq_all / p.splits - qa;
  // the K-range's 128-blocks [bq0, bq0 + nbk): wave w of a projection takes
  // blocks w, w + 4, w + 8, w + 12 (16 lanes each)
  const int bq0 = qa >> 1, nbk = ((qa + nq + 1) >> 1) - bq0;
  const int pblk = pair + 4 * (lane >> 4);
  const bool pwave = pair < nbk;  // uniform
  Pro8In pin;
  if (pwave) {
    const size_t off = (size_t)(bq0 + min(pblk, nbk - 1)) * 128 + (lane & 15) * 8;
    pin = pro8_load(dp.x, dp.x_dtype, (size_t)row * dp.in + off,
                    dp.gu_suh + ((size_t)e * 2 + proj) * dp.in + off);
  }
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7;
  const int tpe = p.width / 16;
  const size_t qstride = (size_t)4 * p.tn_total * 8 * K;
  const int tcol = (proj * p.experts + e) * tpe + cblk * 8 + 2 * pair + hsel;
  const uint32_t* tp =
      p.trellis + ((size_t)(4 * qa + g) * p.tn_total + tcol) * (8 * K) + (size_t)j * K;
  const int prev_off = j == 0 ? 8 * K - 1 : -1;
  constexpr int D = 2;
  uint32_t setA[D][K + 1], setB[D][K + 1];
  const int qlast = nq - 1;
  auto fetch = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      load_slice_prev<K>(tp + (size_t)min(qbase + d, qlast) * qstride, prev_off, set[d]);
  };
  fetch(setA, 0);
  if (pwave) pro8_finish(pin, dp.x_dtype, xs[proj] + pblk * 128 + (lane & 15) * 8, pblk < nbk, lane);
  __syncthreads();
  const _Float16* xrow = (const _Float16*)xs[proj] + (qa - 2 * bq0) * 64 + 16 * g;
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int q = qbase + d;
      if (q < nq) {  // uniform
        const half8 a0 = *(const half8*)(xrow + q * 64);
        const half8 a1 = *(const half8*)(xrow + q * 64 + 8);
        qmv_step_prev<K, CB>(set[d], a0, a1, acc0, acc1);
      }
    }
  };
  for (int q0 = 0; q0 < nq; q0 += 2 * D) {
    fetch(setB, q0 + D);
    compute(setA, q0);
    fetch(setA, q0 + 2 * D);
    compute(setB, q0 + D);
  }
  // accumulator lane l < 16 holds row 0 at column 32*pair + 16*(l/8) + l%8 (+8: acc1)
  const int col = 32 * pair + 16 * (lane >> 3) + (lane & 7);
  if (p.splits == 1) {
    if (g == 0) {
      red[proj][col] = acc0[0];
      red[proj][col + 8] = acc1[0];
    }
    __syncthreads();
    if (wave == 0)
      moe_finish_row<true>(p, e, slot, cblk, red[0][lane], red[0][lane + 64], red[1][lane],
                           red[1][lane + 64], lane);
    return;
  }
  float* part = p.partials + ((size_t)split * 2 + proj) * p.slots_pad * p.width;
  if (g == 0) {
    float* dst = part + (size_t)slot * p.width + cblk * 128 + col;
    store_coherent(dst, acc0[0]);
    store_coherent(dst + 8, acc1[0]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t* counter = dp.counters + (size_t)slot * p.col_blocks + cblk;
  if (threadIdx.x == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == (uint32_t)(p.splits - 1);
  }
  __syncthreads();
  if (!s_last) return;  // uniform
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (wave != 0) return;
  // split sums in split order (as moe_mm_kernel's last arriver)
  constexpr int kChunk = kSplitChunk / 2;
  float v[2][2] = {};
  for (int s0 = 0; s0 < p.splits; s0 += kChunk) {
    float t[kChunk][2][2];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int s = min(s0 + c, p.splits - 1);  // clamped: always a written split
#pragma unroll
      for (int pj = 0; pj < 2; ++pj) {
        const float* src =
            p.partials + ((size_t)(s * 2 + pj) * p.slots_pad + slot) * p.width + cblk * 128;
        t[c][pj][0] = load_coherent(src + lane);
        t[c][pj][1] = load_coherent(src + lane + 64);
      }
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c)
#pragma unroll
      for (int pj = 0; pj < 2; ++pj) {
        v[pj][0] = add_if(s0 + c < p.splits, v[pj][0], t[c][pj][0]);
        v[pj][1] = add_if(s0 + c < p.splits, v[pj][1], t[c][pj][1]);
      }
  }
  moe_finish_row<true>(p, e, slot, cblk, v[0][0], v[0][1], v[1][0], v[1][1], lane);
}

// Down + weighted top-k sum: grid slots * (in / 128) * splits, 256 threads.
template <int K, int CB>
__global__ __launch_bounds__(256) void moe_dec_down_kernel(MoeDecParams dp) {
  const MoeMmParams& p = dp.m;
  __shared__ float red[128];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pair = wave;
  const int per_slot = p.col_blocks * p.splits;
  const int slot = blockIdx.x / per_slot, rem = blockIdx.x - slot * per_slot;
  const int cblk = rem / p.splits, split = rem - cblk * p.splits;
  const uint32_t eu = dp.selected[slot];
  if (eu >= (uint32_t)p.experts) {  // uniform: the slot adds nothing
    // ... and when none of its token's slots is in the bank, the token's first
    // slot (split 0) writes the zeros no top-k sum will
    const int row = slot / dp.top_k;
    if (slot == row * dp.top_k && split == 0 && wave == 0) {
      bool any = false;
      for (int t = 0; t < dp.top_k; ++t)
        any = any || dp.selected[(size_t)row * dp.top_k + t] < (uint32_t)p.experts;
      if (!any) {
        const size_t o = (size_t)row * p.width + cblk * 128 + lane;
        store_reduced(dp.y, p.scores_dtype, o, 0.f);
        store_reduced(dp.y, p.scores_dtype, o + 64, 0.f);
      }
    }
    return;
  }
  const int e = (int)eu, row = slot / dp.top_k;
  const int nq_all = p.k_in >> 6;
  const int qa = split * nq_all / p.splits, nq = (split + 1) * nq_all / p.splits - qa;
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7;
  const int tpe = p.width / 16;
  const size_t qstride = (size_t)4 * p.tn_total * 8 * K;
  const int tcol = e * tpe + cblk * 8 + 2 * pair + hsel;
  const uint32_t* tp =
      p.trellis + ((size_t)(4 * qa + g) * p.tn_total + tcol) * (8 * K) + (size_t)j * K;
  const int prev_off = j == 0 ? 8 * K - 1 : -1;
  const _Float16* xrow = (const _Float16*)p.xa + (size_t)slot * p.k_in + qa * 64 + 16 * g;
  constexpr int D = 2;
  uint32_t setA[D][K + 1], setB[D][K + 1];
  const int qlast = nq - 1;
  auto fetch = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      load_slice_prev<K>(tp + (size_t)min(qbase + d, qlast) * qstride, prev_off, set[d]);
  };
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int q = qbase + d;
      if (q < nq) {  // uniform
        const half8 a0 = *(const half8*)(xrow + q * 64);
        const half8 a1 = *(const half8*)(xrow + q * 64 + 8);
        qmv_step_prev<K, CB>(set[d], a0, a1, acc0, acc1);
      }
    }
  };
  fetch(setA, 0);
  for (int q0 = 0; q0 < nq; q0 += 2 * D) {
    fetch(setB, q0 + D);
    compute(setA, q0);
    fetch(setA, q0 + 2 * D);
    compute(setB, q0 + D);
  }
  const int col = 32 * pair + 16 * (lane >> 3) + (lane & 7);
  float s0v, s1v;  // the slot's column sums (wave 0 of the finishing workgroup)
  if (p.splits == 1) {
    if (g == 0) {
      red[col] = acc0[0];
      red[col + 8] = acc1[0];
    }
    __syncthreads();
    if (wave != 0) return;
    s0v = red[lane];
    s1v = red[lane + 64];
  } else {
    float* part = p.partials + (size_t)split * p.slots_pad * p.width;
    if (g == 0) {
      float* dst = part + (size_t)slot * p.width + cblk * 128 + col;
      store_coherent(dst, acc0[0]);
      store_coherent(dst + 8, acc1[0]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t* counter = dp.counters + (size_t)slot * p.col_blocks + cblk;
    if (threadIdx.x == 0) {
      const uint32_t old =
          __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = old == (uint32_t)(p.splits - 1);
    }
    __syncthreads();
    if (!s_last) return;  // uniform
    if (threadIdx.x == 0)
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wave != 0) return;
    float v0 = 0.f, v1 = 0.f;
    for (int c0 = 0; c0 < p.splits; c0 += kSplitChunk) {
      float a[kSplitChunk], b[kSplitChunk];
#pragma unroll
      for (int c = 0; c < kSplitChunk; ++c) {
        const int s = min(c0 + c, p.splits - 1);  // clamped: always a written split
        const float* src =
            p.partials + ((size_t)s * p.slots_pad + slot) * p.width + cblk * 128;
        a[c] = load_coherent(src + lane);
        b[c] = load_coherent(src + lane + 64);
      }
#pragma unroll
      for (int c = 0; c < kSplitChunk; ++c) {
        v0 = add_if(c0 + c < p.splits, v0, a[c]);
        v1 = add_if(c0 + c < p.splits, v1, b[c]);
      }
    }
    s0v = v0;
    s1v = v1;
  }
  // wave 0 of the slot's finishing workgroup: its weighted values, then the
  // token's top-k sum by the last of its valid slots
  float z0, z1;
  moe_down_values(p, e, slot, cblk, s0v, s1v, lane, z0, z1);
  float* zrow = dp.zf + (size_t)slot * p.width + cblk * 128;
  store_coherent(zrow + lane, z0);
  store_coherent(zrow + lane + 64, z1);
  __builtin_amdgcn_s_waitcnt(0);  // the stores are acknowledged before the arrival
  uint32_t* rcounter =
      dp.counters + (size_t)p.slots_pad * p.col_blocks + (size_t)row * p.col_blocks + cblk;
  // the token's expert ids (and below its slots' values) are loaded a chunk
  // of kTopChunk slots at a time, not one dependent round trip per slot
  constexpr int kTopChunk = 8;
  int valid = 0;
  for (int t0 = 0; t0 < dp.top_k; t0 += kTopChunk) {
    uint32_t ids[kTopChunk];
#pragma unroll
    for (int c = 0; c < kTopChunk; ++c)
      ids[c] = dp.selected[(size_t)row * dp.top_k + min(t0 + c, dp.top_k - 1)];
#pragma unroll
    for (int c = 0; c < kTopChunk; ++c)
      valid += t0 + c < dp.top_k && ids[c] < (uint32_t)p.experts ? 1 : 0;
  }
  uint32_t old = 0;
  if (lane == 0) {
    old = __hip_atomic_fetch_add(rcounter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)(valid - 1))
      __hip_atomic_store(rcounter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (__builtin_amdgcn_readfirstlane(old) != (uint32_t)(valid - 1)) return;
  // y = sum over the token's valid slots in top-k order (moe_reduce_kernel's
  // order and f32 adds), stored as f16 or f32
  moe_token_sum(p, dp.selected, dp.top_k, dp.zf, dp.y, row, cblk, lane);
}

}  // namespace exl3
