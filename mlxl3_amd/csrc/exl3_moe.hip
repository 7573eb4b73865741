// MoE SwitchGLU entry points (Exl3SwitchGlu, native/src/moe.rs:611-1085):
// validation as switch_glu_layout (native/src/contracts.rs:4-28) and
// Exl3SwitchGlu::new (moe.rs:835-886), workspace layout, and the four
// launches of the grouped expert path (route plan with the gather of the
// gate/up inputs, gate/up QMM with the fused SwiGLU glue, down QMM with the
// fused per-slot finish, top-k sum).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <new>

#include "../../include/exl3_hip.h"
#include "exl3_launch.hpp"
#include "exl3_moe.hpp"

namespace exl3 {
#define EXL3_MOE_INST(K, CB)                                                          \
  template __global__ void moe_mm_kernel<K, CB, 2, 1>(MoeMmParams);                  \
  template __global__ void moe_mm_kernel<K, CB, 1, 1>(MoeMmParams);                  \
  template __global__ void moe_mm_kernel<K, CB, 2, 2>(MoeMmParams);                  \
  template __global__ void moe_mm_kernel<K, CB, 1, 2>(MoeMmParams);                  \
  template __global__ void moe_mm_kernel<K, CB, 2, 4>(MoeMmParams);                  \
  template __global__ void moe_mm_kernel<K, CB, 1, 4>(MoeMmParams);                  \
  template __global__ void moe_dec_gu_kernel<K, CB>(MoeDecParams);                   \
  template __global__ void moe_dec_down_kernel<K, CB>(MoeDecParams);
// K = 7 is not a SwitchGLU width (switch_glu_layout rejects it).
EXL3_INST_CB(EXL3_MOE_INST, 1)
EXL3_INST_CB(EXL3_MOE_INST, 2)
EXL3_INST_CB(EXL3_MOE_INST, 3)
EXL3_INST_CB(EXL3_MOE_INST, 4)
EXL3_INST_CB(EXL3_MOE_INST, 5)
EXL3_INST_CB(EXL3_MOE_INST, 6)
EXL3_INST_CB(EXL3_MOE_INST, 8)
template __global__ void moe_route_kernel<true>(MoePlanParams, MoeGatherParams);
template __global__ void moe_route_kernel<false>(MoePlanParams, MoeGatherParams);
template __global__ void moe_reduce_kernel<true>(const void*, int, const uint32_t*, int, int, int,
                                                 void*);
template __global__ void moe_reduce_kernel<false>(const void*, int, const uint32_t*, int, int,
                                                  int, void*);
}  // namespace exl3

using namespace exl3;

#ifndef __HIP_DEVICE_COMPILE__

typedef void (*MoeKernel)(MoeMmParams);
#define EXL3_MOE_ROW(N, MB, K) \
  {moe_mm_kernel<K, 0, N, MB>, moe_mm_kernel<K, 1, N, MB>, moe_mm_kernel<K, 2, N, MB>}
#define EXL3_MOE_TABLE(N, MB)                                                             \
  {EXL3_MOE_ROW(N, MB, 1), EXL3_MOE_ROW(N, MB, 2), EXL3_MOE_ROW(N, MB, 3),               \
   EXL3_MOE_ROW(N, MB, 4), EXL3_MOE_ROW(N, MB, 5), EXL3_MOE_ROW(N, MB, 6),               \
   {nullptr, nullptr, nullptr}, EXL3_MOE_ROW(N, MB, 8)}
// [block rows 16, 32, 64][K-1][codebook]
static const MoeKernel kGateUp[3][8][3] = {EXL3_MOE_TABLE(2, 1), EXL3_MOE_TABLE(2, 2),
                                           EXL3_MOE_TABLE(2, 4)};
static const MoeKernel kDown[3][8][3] = {EXL3_MOE_TABLE(1, 1), EXL3_MOE_TABLE(1, 2),
                                         EXL3_MOE_TABLE(1, 4)};
typedef void (*MoeDecKernel)(MoeDecParams);
#define EXL3_DEC_ROW(F, K) {F<K, 0>, F<K, 1>, F<K, 2>}
#define EXL3_DEC_TABLE(F)                                                                   \
  {EXL3_DEC_ROW(F, 1), EXL3_DEC_ROW(F, 2), EXL3_DEC_ROW(F, 3), EXL3_DEC_ROW(F, 4),         \
   EXL3_DEC_ROW(F, 5), EXL3_DEC_ROW(F, 6), {nullptr, nullptr, nullptr}, EXL3_DEC_ROW(F, 8)}
static const MoeDecKernel kDecGateUp[8][3] = EXL3_DEC_TABLE(moe_dec_gu_kernel);
static const MoeDecKernel kDecDown[8][3] = EXL3_DEC_TABLE(moe_dec_down_kernel);

struct exl3_moe {
  const uint16_t *gu_trellis, *gu_suh, *gu_svh;
  const uint16_t *down_trellis, *down_suh, *down_svh;
  int in, hidden, experts, top_k, k, cb;
  int gelu;            // GluActivation::Gelu (forward_gelu) instead of SiLU
  int logical_hidden;  // GELU: GEGLU outputs of columns >= logical_hidden are zero
  int force_splits;    // EXL3_MOE_SPLITS at create (0: by slot count)
  void* owned;       // device memory freed with the handle (checkpoint loads), or null
};

void exl3::adopt_device_memory(exl3_moe* h, void* mem) { h->owned = mem; }

// The largest bank the route launch's LDS histogram holds (3 ints per expert).
static constexpr int kMoeMaxExperts = 4096;
static constexpr size_t kMoeAlign = 256;
static size_t moe_align(size_t v) { return (v + kMoeAlign - 1) / kMoeAlign * kMoeAlign; }

namespace {
// K-splits of an expert QMM.  The block count is known only on the device;
// min(slots, E) + slots/16 bounds it, and the split count aims at about 512
// workgroups with at least two 64-row K-steps per split.
int moe_splits(const exl3_moe* h, int64_t slots, int block_rows, int k_in, int col_blocks) {
  if (h->force_splits > 0) return std::min(h->force_splits, k_in / 64);
  const int64_t blocks = std::min<int64_t>(slots, h->experts) + slots / block_rows;
  const int64_t base = std::max<int64_t>(1, blocks * col_blocks);
  int s = (int)std::min<int64_t>((512 + base - 1) / base, 16);
  return std::max(1, std::min(s, k_in / 128));
}

// The small-row path (decode): up to this many routed slots run as two
// launches, one workgroup row per slot (moe_dec_*_kernel), where the grouped
// path's four launches cost more than the weight reuse it offers (C4 bank,
// top-8, same box: 1 token 29.4 -> 24.4 us, 4 tokens 46.3 -> 40.9, 8 tokens
// 64.7 -> 60.6 with the first split rule).
static constexpr int64_t kMoeSmallSlots = 64;

// K-splits of a small-row projection, at most 30 steps of 64 inputs each (the
// gate/up prologue holds 16 blocks of 128 inputs).  Gate/up: ranges of about
// 8 steps; down: about 384 workgroups over slots x column blocks with at least
// 2 steps per range.  Measured on the C4 bank, top-8, same box (us, 1 / 4
// tokens): gate/up splits 2: 29.0 / 44.6, 4: 24.4 / 40.9, 8: 25.8 / 47.3, 16:
// 27.8 / 59.6; down splits 1: 27.4 / 44.6, 2: 25.8 / 45.9, 4: 25.7 / 46.7, 12:
// 30.8 / 61.7 (the down rule's picks: 3 / 1).  EXL3_MOE_SPLITS at create pins
// both (then the small-row and grouped paths give equal outputs).
int moe_small_splits(const exl3_moe* h, int64_t slots, int k_in, int col_blocks, bool gate_up) {
  const int nq = k_in / 64;
  const int lo = (nq + 29) / 30;
  if (h->force_splits > 0) return std::max(lo, std::min(h->force_splits, nq));
  int s;
  if (gate_up) {
    s = (nq + 4) / 8;
  } else {
    const int64_t base = std::max<int64_t>(1, slots * col_blocks);
    s = (int)((384 + base / 2) / base);
    s = std::min(s, std::max(1, nq / 2));
  }
  return std::max(std::max(s, 1), lo);
}

// Workspace layout for `slots` = rows * top_k routed slots.
struct MoeLayout {
  size_t counts, rank, sorted, expert_count, table, counters, xgu, xd, z, partials, total;
  int max_blocks, ncounters, splits_gu, splits_down, block_rows;
  int small, small_gu, small_down;  // small-row path and its split counts
};

bool moe_layout(const exl3_moe* h, int64_t rows, MoeLayout& L) {
  if (rows < 1) return false;
  const int64_t slots = rows * h->top_k;
  if (slots > (int64_t)1 << 24) return false;
  // Rows per block by the average rows an expert sees: 16 below 8, 32 up to
  // 24 (most experts then fit one block, and the 32-row kernel's 113 VGPRs
  // leave room for two workgroups per CU where the 64-row kernel's ~170 allow
  // one: 185 -> 162 us on the 256-token top-8 bank of 128 experts), 64 above
  // (fewer blocks, so fewer decodes of each expert's weights).
  const int64_t E = h->experts;
  L.block_rows = slots < 8 * E ? 16 : slots <= 24 * E ? 32 : kMoeMaxBlockRows;
  if (const char* env = getenv("EXL3_MOE_BLOCK_ROWS")) {
    const int v = atoi(env);
    if (v == 16 || v == 32 || v == 64) L.block_rows = v;
  }
  // each routed expert's last block may be partial: sum ceil(c_e/b) <=
  // slots/b + (experts routed) <= slots/b + min(E, slots).  The expert QMM
  // grids are sized by this bound, so a decode call (8 slots) launches the
  // workgroups of 9 blocks, not of E + 1 that exit at once.
  const int64_t max_blocks = slots / L.block_rows + std::min<int64_t>(h->experts, slots) + 1;
  const int64_t ncounters = max_blocks * (std::max(h->hidden, h->in) / 128);
  if (ncounters > INT32_MAX) return false;
  L.max_blocks = (int)max_blocks;
  L.ncounters = (int)ncounters;
  L.splits_gu = moe_splits(h, slots, L.block_rows, h->in, h->hidden / 128);
  L.splits_down = moe_splits(h, slots, L.block_rows, h->hidden, h->in / 128);
  // small-row path: its arrival counters (gate/up, down, top-k sums) must fit
  // the workspace's counter region
  const int64_t small_counters =
      slots * (h->hidden / 128 + h->in / 128) + rows * (h->in / 128);
  L.small = slots <= kMoeSmallSlots && !getenv("EXL3_MOE_GROUPED") &&
            small_counters * 4 <= (int64_t)kWorkspaceCounterBytes;
  L.small_gu = L.small ? moe_small_splits(h, slots, h->in, h->hidden / 128, true) : 0;
  L.small_down = L.small ? moe_small_splits(h, slots, h->hidden, h->in / 128, false) : 0;
  if (L.small) {  // tuning overrides of the small-row split counts
    if (const char* env = getenv("EXL3_MOE_SMALL_GU"))
      L.small_gu = std::max((h->in / 64 + 29) / 30, std::min(atoi(env), h->in / 64));
    if (const char* env = getenv("EXL3_MOE_SMALL_DOWN"))
      L.small_down = std::max((h->hidden / 64 + 29) / 30, std::min(atoi(env), h->hidden / 64));
  }
  size_t off = kWorkspaceCounterBytes;  // the shared counter region stays untouched
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = moe_align(off + bytes);
    return at;
  };
  L.counts = take(2 * sizeof(int));
  L.rank = take((size_t)slots * sizeof(int));
  L.sorted = take((size_t)slots * sizeof(int));
  L.expert_count = take((size_t)h->experts * sizeof(int));
  L.table = take((size_t)L.max_blocks * sizeof(int4));
  L.counters = take((size_t)L.ncounters * sizeof(uint32_t));
  L.xgu = take((size_t)2 * slots * h->in * sizeof(uint16_t));
  L.xd = take((size_t)slots * h->hidden * sizeof(uint16_t));
  L.z = take((size_t)slots * h->in * sizeof(float));  // f32 for f32 / bf16 scores
  const int sgu = std::max(L.splits_gu, L.small_gu), sdn = std::max(L.splits_down, L.small_down);
  const size_t pgu = sgu > 1 ? (size_t)sgu * 2 * slots * h->hidden : 0;
  const size_t pdn = sdn > 1 ? (size_t)sdn * slots * h->in : 0;
  L.partials = take(std::max(pgu, pdn) * sizeof(float));
  L.total = off;
  return true;
}
}  // namespace

// The small-row path: gate/up (+ SwiGLU glue) and down (+ finish and top-k
// sum) as two launches over the slots (moe_dec_*_kernel).
static int moe_forward_small(const exl3_moe* h, const MoeLayout& L, const void* x, int x_type,
                             int64_t rows, const uint32_t* selected, const void* scores,
                             int scores_type, void* y, char* ws, hipStream_t s) {
  const MoeDecKernel gateup = kDecGateUp[h->k - 1][h->cb], down = kDecDown[h->k - 1][h->cb];
  if (!gateup || !down) return fail(EXL3_EUNSUPPORTED, "no SwitchGLU kernel for K=%d", h->k);
  const int slots = (int)(rows * h->top_k);
  MoeDecParams dp{};
  MoeMmParams& q = dp.m;
  q.experts = h->experts;
  q.slots_pad = slots;
  q.partials = (float*)(ws + L.partials);
  q.trellis = (const uint32_t*)h->gu_trellis;
  q.tn_total = 2 * h->experts * h->hidden / 16;
  q.k_in = h->in;
  q.width = h->hidden;
  q.col_blocks = h->hidden / 128;
  q.splits = L.small_gu;
  q.gu_svh = h->gu_svh;
  q.down_suh = h->down_suh;
  q.xd = (uint16_t*)(ws + L.xd);
  q.gelu = h->gelu;
  q.logical_hidden = h->logical_hidden;
  q.down_svh = h->down_svh;
  q.scores = scores;
  q.scores_dtype = scores_type;
  dp.x = x;
  dp.x_dtype = x_type;
  dp.top_k = h->top_k;
  dp.in = h->in;
  dp.selected = selected;
  dp.gu_suh = h->gu_suh;
  dp.counters = (uint32_t*)ws;  // the workspace's counter region
  dp.zf = (float*)(ws + L.z);
  dp.y = y;
  if (int rc = launch_gate("moe gate/up")) return rc;
  gateup<<<(unsigned)(slots * q.col_blocks * q.splits), 512, 0, s>>>(dp);
  if (int rc = check_launch("moe gate/up")) return rc;
  MoeDecParams dd = dp;
  dd.m.trellis = (const uint32_t*)h->down_trellis;
  dd.m.tn_total = h->experts * h->in / 16;
  dd.m.k_in = h->hidden;
  dd.m.width = h->in;
  dd.m.col_blocks = h->in / 128;
  dd.m.splits = L.small_down;
  dd.m.xa = q.xd;
  dd.counters = dp.counters + (size_t)slots * q.col_blocks;
  if (int rc = launch_gate("moe down")) return rc;
  down<<<(unsigned)(slots * dd.m.col_blocks * dd.m.splits), 256, 0, s>>>(dd);
  return check_launch("moe down");
}

extern "C" {

int exl3_moe_create(const uint16_t* gu_trellis, const uint16_t* gu_suh, const uint16_t* gu_svh,
                    const uint16_t* down_trellis, const uint16_t* down_suh,
                    const uint16_t* down_svh, int32_t in, int32_t hidden, int32_t experts,
                    int32_t top_k, int32_t k, int32_t cb, exl3_moe** out_handle) {
  if (!out_handle) return fail(EXL3_EINVAL, "out_handle is null");
  *out_handle = nullptr;
  if (experts <= 0 || top_k <= 0 || top_k > experts || in <= 0 || hidden <= 0 || in % 128 ||
      hidden % 128 || k < 1 || k > 8 || k == 7 ||
      (int64_t)experts * hidden > INT32_MAX || (int64_t)experts * in > INT32_MAX)
    return fail(EXL3_EINVAL, "invalid or overflowing SwitchGLU dimensions");
  if (cb < 0 || cb > 2) return fail(EXL3_EINVAL, "invalid EXL3 codebook %d", cb);
  if (!gu_trellis || !gu_suh || !gu_svh || !down_trellis || !down_suh || !down_svh)
    return fail(EXL3_EINVAL, "SwitchGLU trellis/scales disagree");
  if (experts > kMoeMaxExperts)
    return fail(EXL3_EUNSUPPORTED, "SwitchGLU banks of more than %d experts are not supported",
                kMoeMaxExperts);
  exl3_moe* h = new (std::nothrow) exl3_moe;
  if (!h) return fail(EXL3_ENOMEM, "out of host memory");
  *h = exl3_moe{gu_trellis, gu_suh, gu_svh, down_trellis, down_suh, down_svh,
                in,         hidden, experts, top_k,       k,        cb,
                0,          hidden, 0,       nullptr};
  if (const char* env = getenv("EXL3_MOE_SPLITS")) h->force_splits = std::max(0, atoi(env));
  *out_handle = h;
  return EXL3_OK;
}

int exl3_moe_create_gelu(const uint16_t* gu_trellis, const uint16_t* gu_suh,
                         const uint16_t* gu_svh, const uint16_t* down_trellis,
                         const uint16_t* down_suh, const uint16_t* down_svh, int32_t in,
                         int32_t hidden, int32_t experts, int32_t top_k, int32_t k, int32_t cb,
                         int32_t logical_hidden, exl3_moe** out_handle) {
  if (!out_handle) return fail(EXL3_EINVAL, "out_handle is null");
  *out_handle = nullptr;
  // forward_gelu zeroes the columns from logical_hidden on only when it is
  // below hidden (moe.rs:1125-1137); a width of zero or less has no meaning
  if (logical_hidden <= 0) return fail(EXL3_EINVAL, "invalid logical GLU width");
  if (int rc = exl3_moe_create(gu_trellis, gu_suh, gu_svh, down_trellis, down_suh, down_svh, in,
                               hidden, experts, top_k, k, cb, out_handle))
    return rc;
  (*out_handle)->gelu = 1;
  (*out_handle)->logical_hidden = std::min(logical_hidden, hidden);
  return EXL3_OK;
}

int32_t exl3_moe_in_features(const exl3_moe* h) { return h ? h->in : 0; }
int32_t exl3_moe_hidden_features(const exl3_moe* h) { return h ? h->hidden : 0; }

void exl3_moe_destroy(exl3_moe* h) {
  if (h && h->owned) (void)hipFree(h->owned);
  delete h;
}

size_t exl3_moe_workspace_bytes(const exl3_moe* h, int64_t rows) {
  MoeLayout L;
  if (!h || !moe_layout(h, rows, L)) return 0;
  return L.total;
}

int exl3_swiglu_down_input(const float* gate_up, const uint16_t* gu_svh, const uint16_t* down_suh,
                           const uint32_t* selected, int64_t slots, int32_t hidden,
                           int32_t experts, uint16_t* xhat, void* stream) {
  // glu_down_input's checks (moe.rs:459-467)
  if (slots <= 0 || slots > INT32_MAX || hidden <= 0 || hidden % 128)
    return fail(EXL3_EINVAL, "invalid fused SwiGLU dimensions");
  if (hidden / 128 > 65535)  // grid.y holds the column blocks
    return fail(EXL3_EUNSUPPORTED, "SwiGLU width %d is too large", hidden);
  if (experts <= 0 || !gu_svh || !down_suh || !selected)
    return fail(EXL3_EINVAL, "invalid fused SwiGLU scales/routes");
  if (!gate_up || !xhat) return fail(EXL3_EINVAL, "null SwiGLU buffer");
  MoeMmParams q{};
  q.width = hidden;
  q.experts = experts;
  q.gu_svh = gu_svh;
  q.down_suh = down_suh;
  q.xd = xhat;
  swiglu_down_input_kernel<<<dim3((unsigned)slots, hidden / 128), 64, 0, (hipStream_t)stream>>>(
      q, gate_up, selected);
  return check_launch("swiglu_down_input launch");
}

int exl3_finish_and_reduce(const float* raw, const uint16_t* svh, const void* scores,
                           int32_t scores_type, int64_t rows, int32_t top_k, int32_t width,
                           void* y, void* stream) {
  // finish_and_reduce's checks (moe.rs:596-602)
  if (rows <= 0 || rows > INT32_MAX || top_k <= 0 || width <= 0 || width % 128)
    return fail(EXL3_EINVAL, "invalid expert reduction dimensions");
  if (width / 128 > 65535)  // grid.y holds the column blocks
    return fail(EXL3_EUNSUPPORTED, "expert reduction width %d is too large", width);
  if (rows * (int64_t)top_k > INT32_MAX)
    return fail(EXL3_EINVAL, "invalid expert reduction dimensions");
  if (!raw || !svh || !scores || !y) return fail(EXL3_EINVAL, "null expert reduction buffer");
  if (scores_type != EXL3_F16 && scores_type != EXL3_F32 && scores_type != EXL3_BF16)
    return fail(EXL3_EINVAL, "unsupported score dtype code %d", scores_type);
  finish_and_reduce_kernel<<<dim3((unsigned)rows, width / 128), 64, 0, (hipStream_t)stream>>>(
      raw, svh, scores, scores_type, top_k, width, y);
  return check_launch("finish_and_reduce launch");
}

static bool valid_dtype(int dt) { return dt == EXL3_F16 || dt == EXL3_F32 || dt == EXL3_BF16; }

int exl3_moe_forward(const exl3_moe* h, const void* x, int32_t x_type, int64_t rows,
                     const uint32_t* selected, const void* scores, int32_t scores_type, void* y,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!h) return fail(EXL3_EINVAL, "handle is null");
  if (rows < 1 || !x || !selected || !scores || !y)
    return fail(EXL3_EINVAL, "invalid SwitchGLU input/routes");
  if (!valid_dtype(x_type) || !valid_dtype(scores_type))
    return fail(EXL3_EINVAL, "unsupported dtype codes %d (x), %d (scores)", x_type, scores_type);
  MoeLayout L;
  if (!moe_layout(h, rows, L)) return fail(EXL3_EINVAL, "MoE slot overflow");
  if (!workspace || workspace_bytes < L.total)
    return fail(EXL3_EINVAL, "workspace too small: need %zu bytes, got %zu", L.total,
                workspace_bytes);
  const int mbi = L.block_rows == kMoeMaxBlockRows ? 2 : L.block_rows == 32 ? 1 : 0;
  const MoeKernel gateup = kGateUp[mbi][h->k - 1][h->cb], down = kDown[mbi][h->k - 1][h->cb];
  if (!gateup || !down) return fail(EXL3_EUNSUPPORTED, "no SwitchGLU kernel for K=%d", h->k);
  const int64_t wide = (int64_t)(L.max_blocks + 7) * (std::max(h->in, h->hidden) / 128) *
                       std::max(L.splits_gu, L.splits_down);
  if (wide * 512 >= ((int64_t)1 << 31))
    return fail(EXL3_EUNSUPPORTED, "SwitchGLU launch of %lld rows is too large", (long long)rows);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int slots = (int)(rows * h->top_k);
  if (L.small && (((uintptr_t)x | (uintptr_t)h->gu_suh) & 15) == 0)
    return moe_forward_small(h, L, x, x_type, rows, selected, scores, scores_type, y, ws, s);

  MoePlanParams pp;
  pp.selected = selected;
  pp.slots = slots;
  pp.experts = h->experts;
  pp.rank = (int*)(ws + L.rank);
  pp.sorted_slot = (int*)(ws + L.sorted);
  pp.table = (int4*)(ws + L.table);
  pp.counts = (int*)(ws + L.counts);
  pp.expert_count = (int*)(ws + L.expert_count);
  pp.counters = (uint32_t*)(ws + L.counters);
  pp.ncounters = L.ncounters;
  pp.block_rows = L.block_rows;
  MoeGatherParams gp;
  gp.x = x;
  gp.x_dtype = x_type;
  gp.in = h->in;
  gp.top_k = h->top_k;
  gp.slots = slots;
  gp.experts = h->experts;
  gp.selected = selected;
  gp.gu_suh = h->gu_suh;
  gp.xgu = (uint16_t*)(ws + L.xgu);
  const unsigned route_wgs =
      1u + (unsigned)((2 * (int64_t)slots * ((h->in / 128 + 7) / 8) + 3) / 4);
  const size_t plan_lds = (3 * (size_t)h->experts + 1) * sizeof(int);
  if (int rc = launch_gate("moe plan")) return rc;
  if ((((uintptr_t)x | (uintptr_t)h->gu_suh) & 15) == 0)
    moe_route_kernel<true><<<route_wgs, 256, plan_lds, s>>>(pp, gp);
  else
    moe_route_kernel<false><<<route_wgs, 256, plan_lds, s>>>(pp, gp);
  if (int rc = check_launch("moe plan")) return rc;

  MoeMmParams q{};
  q.experts = h->experts;
  q.table = pp.table;
  q.counts = pp.counts;
  q.sorted_slot = pp.sorted_slot;
  q.slots_pad = slots;
  q.partials = (float*)(ws + L.partials);
  q.counters = pp.counters;
  // gate/up: input width `in`, per-expert output `hidden`
  q.trellis = (const uint32_t*)h->gu_trellis;
  q.tn_total = 2 * h->experts * h->hidden / 16;
  q.k_in = h->in;
  q.width = h->hidden;
  q.col_blocks = h->hidden / 128;
  q.splits = L.splits_gu;
  q.xa = gp.xgu;
  q.a_rows = pp.sorted_slot;
  q.gu_svh = h->gu_svh;
  q.down_suh = h->down_suh;
  q.xd = (uint16_t*)(ws + L.xd);
  q.gelu = h->gelu;
  q.logical_hidden = h->logical_hidden;
  const int grid_blocks = (L.max_blocks + 7) / 8 * 8;  // whole blocks per XCD
  // down: input width `hidden`, per-expert output `in`
  MoeMmParams d = q;
  d.trellis = (const uint32_t*)h->down_trellis;
  d.tn_total = h->experts * h->in / 16;
  d.k_in = h->hidden;
  d.width = h->in;
  d.col_blocks = h->in / 128;
  d.splits = L.splits_down;
  d.xa = q.xd;
  d.a_rows = nullptr;
  d.down_svh = h->down_svh;
  d.scores = scores;
  d.scores_dtype = scores_type;
  d.z = ws + L.z;
  gateup<<<grid_blocks * q.col_blocks * q.splits, 512, 0, s>>>(q);
  if (int rc = check_launch("moe gate/up")) return rc;
  down<<<grid_blocks * d.col_blocks * d.splits, 256, 0, s>>>(d);
  if (int rc = check_launch("moe down")) return rc;

  const dim3 rgrid((unsigned)rows, (h->in + 2047) / 2048);
  if (((uintptr_t)y & 15) == 0)
    moe_reduce_kernel<true><<<rgrid, 256, 0, s>>>(d.z, scores_type, selected, h->experts,
                                                   h->top_k, h->in, y);
  else
    moe_reduce_kernel<false><<<rgrid, 256, 0, s>>>(d.z, scores_type, selected, h->experts,
                                                    h->top_k, h->in, y);
  return check_launch("moe reduce");
}

}  // extern "C"

#endif  // __HIP_DEVICE_COMPILE__
