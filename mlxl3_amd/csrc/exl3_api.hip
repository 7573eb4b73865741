// Host side of the EXL3 library: argument validation (mirroring the checks of
// Exl3Linear::new, native/src/linear.rs:582-607), kernel selection by row
// count, split-K choice, workspace layout and the C ABI of include/exl3_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

#include "../../include/exl3_hip.h"
#include "exl3_launch.hpp"

using namespace exl3;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local char g_error[2048];

int exl3::fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return code;
}

int exl3::check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(EXL3_EDEVICE, "%s: %s", what, hipGetErrorString(e));
  return EXL3_OK;
}

static bool valid_dtype(int dt) { return dt == EXL3_F16 || dt == EXL3_F32 || dt == EXL3_BF16; }

// ---------------------------------------------------------------------------
// handles
// ---------------------------------------------------------------------------
struct exl3_linear {
  const uint16_t* trellis;
  const uint16_t* suh;
  const uint16_t* svh;
  const uint16_t* bias;
  int in, out, k, cb;
  int qmv_splits;
  int qmv_kw;  // K-parts per column pair inside a workgroup (1, 2, 4)
  void* owned;  // device memory freed with the handle (checkpoint loads), or null
};

void exl3::adopt_device_memory(exl3_linear* h, void* mem) { h->owned = mem; }

static constexpr int kQmvMaxRows = 16;
static constexpr size_t kAlign = 256;
static size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// QMV launch shape.  Workgroups: out/128 column blocks x `splits` K-ranges
// (global split-K, reduced by the last workgroup of a column block); inside a
// workgroup KW waves per column pair split the K-range again (LDS reduction).
// Target: about two workgroups of 4*KW waves per CU, at most 8 Hadamard
// blocks (1024 rows) per K-range so xhat fits LDS.  EXL3_QMV_SPLITS and
// EXL3_QMV_KW override (tuning).
static void choose_qmv_shape(int in, int out, int* splits_out, int* kw_out) {
  const int nb = in / 128, col_blocks = out / 128;
  const int min_splits = (nb + 7) / 8;
  int kw = 1;
  if (const char* env = getenv("EXL3_QMV_KW")) {
    int v = atoi(env);
    if (v == 1 || v == 2 || v == 4) kw = v;
  }
  const int target_wgs = 448;
  int s = (target_wgs + col_blocks - 1) / col_blocks;
  if (const char* env = getenv("EXL3_QMV_SPLITS")) {
    int v = atoi(env);
    if (v >= 1) s = v;
  }
  s = std::max(1, std::min(std::max(s, min_splits), nb));
  *splits_out = s;
  *kw_out = kw;
}

// QMM launch shape: rows per workgroup 64*MB and global K-splits.  One
// workgroup of 8 waves fills a CU (two waves per SIMD), so the cost model
// counts rounds of 256 workgroups times K-steps per split times the step
// time, which is the larger of the consumers' MFMA time (16*MB MFMAs of 16
// cycles) and the producers' decode time (~720 cycles), plus ~100 cycles of
// barrier; a split adds its f32 partial traffic (written and read back at
// ~5 TB/s, i.e. ~0.4 cycles per byte at 2.1 GHz).  Splits are only used while
// the output tiles alone fill fewer than 192 CUs, so at most 256 tile
// counters are ever needed.  EXL3_QMM_MB and EXL3_QMM_SPLITS override.
static constexpr int kTileCounters = 256;

struct QmmShape {
  int mb, mtiles, splits;
};

static QmmShape choose_qmm_shape(int in, int out, int64_t rows) {
  const int col_blocks = out / 128, nq = in / 64;
  int force_mb = 0, force_splits = 0;
  if (const char* env = getenv("EXL3_QMM_MB")) {
    int v = atoi(env);
    if (v == 1 || v == 2 || v == 4) force_mb = v;
  }
  if (const char* env = getenv("EXL3_QMM_SPLITS")) force_splits = std::max(0, atoi(env));
  QmmShape best{4, 1, 1};
  double best_cost = 1e300;
  for (int mb : {4, 2, 1}) {
    if (force_mb && mb != force_mb) continue;
    const int64_t mt = (rows + 64 * mb - 1) / (64 * mb);
    const int64_t base = mt * col_blocks;
    int splits = 1;
    if (base < 192) splits = (int)std::min<int64_t>((256 + base - 1) / base, 8);
    if (force_splits) splits = force_splits;
    splits = std::max(1, std::min(splits, std::max(1, nq / 4)));
    if (splits > 1 && base > kTileCounters) splits = 1;
    const int64_t rounds = (base * splits + 255) / 256;
    const double step = std::max(256.0 * mb, 720.0) + 100.0;
    double cost = (double)rounds * ((nq + splits - 1) / splits) * step;
    if (splits > 1) cost += 0.4 * 2.0 * 4.0 * (double)splits * rows * out;
    if (cost < best_cost) {
      best_cost = cost;
      best = QmmShape{mb, (int)mt, splits};
    }
  }
  return best;
}

// Workspace: [tile counters][QMV partials | QMM xhat, partials].  The counter
// region has a fixed size, so one workspace serves QMV and QMM calls in any
// order (every call leaves its counters at zero).
static size_t linear_ws_bytes(const exl3_linear* h, int64_t rows) {
  size_t counters = align_up(sizeof(uint32_t) * (size_t)std::max(h->out / 128, kTileCounters));
  if (rows <= kQmvMaxRows)
    return counters + align_up(sizeof(float) * (size_t)h->qmv_splits * rows * h->out);
  const QmmShape sh = choose_qmm_shape(h->in, h->out, rows);
  size_t partials = sh.splits > 1 ? sizeof(float) * (size_t)sh.splits * rows * h->out : 0;
  return counters + align_up(sizeof(uint16_t) * (size_t)rows * h->in) + align_up(partials);
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
static int linear_forward(const exl3_linear* h, const void* x, int x_type, int64_t rows, void* y,
                          int y_type, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!h) return fail(EXL3_EINVAL, "null EXL3 linear handle");
  if (!x || !y) return fail(EXL3_EINVAL, "null activation pointer");
  if (!valid_dtype(x_type) || !valid_dtype(y_type))
    return fail(EXL3_EINVAL, "unsupported dtype codes %d -> %d", x_type, y_type);
  if (rows < 1) return fail(EXL3_EINVAL, "EXL3 linear input cannot be empty");
  if (rows > (int64_t)INT32_MAX / std::max(h->in, h->out))
    return fail(EXL3_EINVAL, "EXL3 linear input too large: %lld rows", (long long)rows);
  size_t need = linear_ws_bytes(h, rows);
  if (!ws || ws_bytes < need)
    return fail(EXL3_EINVAL, "workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
  uint32_t* counters = (uint32_t*)ws;
  char* after =
      (char*)ws + align_up(sizeof(uint32_t) * (size_t)std::max(h->out / 128, kTileCounters));
  const int kidx = h->k - 1, cb = h->cb;

  if (rows <= kQmvMaxRows) {
    QmvParams p;
    p.trellis = (const uint32_t*)h->trellis;
    p.x = x;
    p.suh = h->suh;
    p.svh = h->svh;
    p.bias = h->bias;
    p.y = y;
    p.partials = (float*)after;
    p.counters = counters;
    p.in = h->in;
    p.out = h->out;
    p.M = (int)rows;
    p.splits = h->qmv_splits;
    p.x_dtype = x_type;
    p.y_dtype = y_type;
    const int nb = h->in / 128;
    int max_blocks = 0;
    for (int s = 0; s < p.splits; ++s)
      max_blocks = std::max(max_blocks, (s + 1) * nb / p.splits - s * nb / p.splits);
    size_t lds = sizeof(uint16_t) * (size_t)rows * max_blocks * 128;
    const int kwi = h->qmv_kw == 4 ? 2 : h->qmv_kw == 2 ? 1 : 0;
    kQmv[kwi][kidx][cb](p, dim3(h->out / 128, p.splits), lds, stream);
    return check_launch("EXL3 QMV launch");
  }

  uint16_t* xhat = (uint16_t*)after;
  launch_prologue(x, x_type, h->suh, h->in, (int)rows, xhat, stream);
  if (int rc = check_launch("EXL3 prologue launch")) return rc;
  const QmmShape sh = choose_qmm_shape(h->in, h->out, rows);
  QmmParams q;
  q.trellis = (const uint32_t*)h->trellis;
  q.xhat = xhat;
  q.svh = h->svh;
  q.bias = h->bias;
  q.y = y;
  q.partials = (float*)((char*)xhat + align_up(sizeof(uint16_t) * (size_t)rows * h->in));
  q.counters = counters;
  q.in = h->in;
  q.out = h->out;
  q.M = (int)rows;
  q.y_dtype = y_type;
  q.col_blocks = h->out / 128;
  q.mtiles = sh.mtiles;
  q.splits = sh.splits;
  const int mbi = sh.mb == 4 ? 2 : sh.mb == 2 ? 1 : 0;
  const int64_t wgs = (int64_t)sh.mtiles * q.col_blocks * sh.splits;
  if (wgs > INT32_MAX) return fail(EXL3_EINVAL, "EXL3 QMM grid too large");
  kQmm[mbi][kidx][cb](q, dim3((unsigned)wgs), stream);
  return check_launch("EXL3 QMM launch");
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* exl3_last_error(void) { return g_error; }

const char* exl3_version(void) { return "exl3-mi355x 0.1 (gfx950)"; }

int exl3_linear_create(const uint16_t* trellis, int32_t in, int32_t out, int32_t k, int32_t cb,
                       const uint16_t* suh, const uint16_t* svh, const uint16_t* bias,
                       exl3_linear** out_handle) {
  if (!out_handle) return fail(EXL3_EINVAL, "null output handle pointer");
  *out_handle = nullptr;
  if (k < 1 || k > 8) return fail(EXL3_EINVAL, "K must be in 1..=8, got %d", k);
  if (cb < 0 || cb > 2) return fail(EXL3_EINVAL, "invalid EXL3 codebook %d", cb);
  if (in <= 0 || out <= 0) return fail(EXL3_EINVAL, "invalid trellis shape");
  if (in % 128 || out % 128)
    return fail(EXL3_EINVAL, "public EXL3 projections require 128-aligned dimensions");
  if (!trellis || !suh || !svh) return fail(EXL3_EINVAL, "null weight pointer");
  exl3_linear* h = new (std::nothrow) exl3_linear;
  if (!h) return fail(EXL3_ENOMEM, "out of host memory");
  h->trellis = trellis;
  h->suh = suh;
  h->svh = svh;
  h->bias = bias;
  h->in = in;
  h->out = out;
  h->k = k;
  h->cb = cb;
  choose_qmv_shape(in, out, &h->qmv_splits, &h->qmv_kw);
  h->owned = nullptr;
  *out_handle = h;
  return EXL3_OK;
}

void exl3_linear_destroy(exl3_linear* handle) {
  if (handle && handle->owned) (void)hipFree(handle->owned);
  delete handle;
}

int32_t exl3_linear_in_features(const exl3_linear* h) { return h ? h->in : 0; }
int32_t exl3_linear_out_features(const exl3_linear* h) { return h ? h->out : 0; }

size_t exl3_linear_workspace_bytes(const exl3_linear* h, int64_t rows) {
  if (!h || rows < 1) return 0;
  return linear_ws_bytes(h, rows);
}

int exl3_workspace_init(void* workspace, size_t bytes, void* stream) {
  if (!workspace || bytes % 4) return fail(EXL3_EINVAL, "workspace must be non-null, 4-byte sized");
  size_t words = bytes / 4;
  unsigned blocks = (unsigned)std::min<size_t>((words + 255) / 256, 4096);
  if (blocks == 0) return EXL3_OK;
  (void)blocks;
  launch_fill_zero((uint32_t*)workspace, words, (hipStream_t)stream);
  return check_launch("workspace init");
}

int exl3_linear_forward(const exl3_linear* h, const void* x, int32_t x_type, int64_t rows, void* y,
                        int32_t y_type, void* workspace, size_t workspace_bytes, void* stream) {
  return linear_forward(h, x, x_type, rows, y, y_type, workspace, workspace_bytes,
                        (hipStream_t)stream);
}

int exl3_group_forward(const exl3_linear* const* parts, int32_t count, const void* x,
                       int32_t x_type, int64_t rows, void* const* ys, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (!parts || !ys || count < 1) return fail(EXL3_EINVAL, "empty EXL3 group");
  for (int i = 0; i < count; ++i) {
    if (!parts[i]) return fail(EXL3_EINVAL, "null EXL3 group member %d", i);
    if (parts[i]->in != parts[0]->in || parts[i]->k != parts[0]->k ||
        parts[i]->cb != parts[0]->cb)
      return fail(EXL3_EINVAL, "EXL3 group members need the same input width, K and codebook");
  }
  for (int i = 0; i < count; ++i) {
    int rc = linear_forward(parts[i], x, x_type, rows, ys[i], x_type, workspace, workspace_bytes,
                            (hipStream_t)stream);
    if (rc) return rc;
  }
  return EXL3_OK;
}

int exl3_decode_tiles(const uint16_t* packed, int64_t tiles, int32_t k, int32_t cb,
                      uint16_t* states, uint16_t* values, void* stream) {
  if (k < 1 || k > 8) return fail(EXL3_EINVAL, "K must be in 1..=8, got %d", k);
  if (cb < 0 || cb > 2) return fail(EXL3_EINVAL, "invalid EXL3 codebook %d", cb);
  if (tiles < 0) return fail(EXL3_EINVAL, "negative tile count");
  if (tiles == 0) return EXL3_OK;
  if (!packed || !values) return fail(EXL3_EINVAL, "null decode buffer");
  int64_t blocks = (tiles * 8 + 255) / 256;
  if (blocks > INT32_MAX) return fail(EXL3_EINVAL, "too many tiles");
  kDecode[k - 1][cb]((const uint32_t*)packed, tiles, states, values, dim3((unsigned)blocks),
                     (hipStream_t)stream);
  return check_launch("EXL3 decode launch");
}

}  // extern "C"

