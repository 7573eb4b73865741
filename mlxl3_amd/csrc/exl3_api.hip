// Host side of the EXL3 library: argument validation (mirroring the checks of
// Exl3Linear::new, native/src/linear.rs:582-607), kernel selection by row
// count, split-K choice, workspace layout and the C ABI of include/exl3_hip.h.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>

#include "../../include/exl3_hip.h"
#include "exl3_launch.hpp"

using namespace exl3;

// ---------------------------------------------------------------------------
// allocation-free workspace (exl3_linear_forward_noalloc)
// ---------------------------------------------------------------------------
// A file-scope device array that stands in for the caller's workspace: its
// first kWorkspaceCounterBytes are the split-K counters (cleared once per
// device, then left at zero by every call), the rest the per-call scratch.
// Every GPU holds its own copy from module load to process exit.  In host code
// the array's name is not a device address: the address comes from
// hipGetSymbolAddress, once per device, and only that pointer is used.
static constexpr size_t kNoAllocBytes = kWorkspaceCounterBytes + ((size_t)32 << 20);
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device

// The scratch address on the current device; on first use the counter region
// is cleared on `stream` (a fill kernel, so the call may be captured).
static int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return fail(EXL3_EDEVICE, "no usable HIP device for the allocation-free workspace");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return fail(EXL3_EDEVICE, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    }
    launch_fill_zero((uint32_t*)ptr, kWorkspaceCounterBytes / 4, stream);
    if (int rc = check_launch("allocation-free workspace init")) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return EXL3_OK;
}

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

// Fault hook: launches whose name contains the armed text fail with
// EXL3_EDEVICE before (launch_gate) or after (check_launch) they are issued,
// so tests can follow the error path, with or without a GPU.  Armed by
// exl3_debug_fail_launch or, at load, by EXL3_FAIL_LAUNCH.
static std::atomic<bool> g_fault_armed{false};
static std::mutex g_fault_mutex;
static std::string g_fault_text;

static bool fault_forced(const char* what) {
  if (!g_fault_armed.load(std::memory_order_relaxed)) return false;
  std::lock_guard<std::mutex> lock(g_fault_mutex);
  return g_fault_armed.load(std::memory_order_relaxed) &&
         std::strstr(what, g_fault_text.c_str()) != nullptr;
}

void exl3_debug_fail_launch(const char* text) {
  std::lock_guard<std::mutex> lock(g_fault_mutex);
  g_fault_text = text ? text : "";
  g_fault_armed.store(text != nullptr, std::memory_order_relaxed);
}

static const bool g_fault_from_env = [] {
  if (const char* env = getenv("EXL3_FAIL_LAUNCH")) exl3_debug_fail_launch(env);
  return true;
}();

int exl3::launch_gate(const char* what) {
  if (fault_forced(what)) return fail(EXL3_EDEVICE, "%s: forced launch failure", what);
  return EXL3_OK;
}

int exl3::check_launch(const char* what) {
  if (fault_forced(what)) return fail(EXL3_EDEVICE, "%s: forced launch failure", what);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(EXL3_EDEVICE, "%s: %s", what, hipGetErrorString(e));
  return EXL3_OK;
}

static bool valid_dtype(int dt) { return dt == EXL3_F16 || dt == EXL3_F32 || dt == EXL3_BF16; }

// Output dtype of a projection (linear.rs:992-995): y.astype(x.dtype) + bias
// with the f16 bias, under MLX's promotion -- bf16 + f16 is f32, f16 + f16
// f16, f32 + f16 f32; without a bias the activation dtype.
static int result_dtype(int x_type, bool has_bias) {
  return has_bias && x_type == EXL3_BF16 ? EXL3_F32 : x_type;
}

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
// Target: about 896 workgroups of 4 waves (3.5 per SIMD), with K-ranges of at
// least 2 Hadamard blocks and at most 8 splits (the last arriver loads every
// split's partials).  Long inputs need more splits: a range holds at most 12
// blocks (xhat of 16 rows in 48 KB of LDS).  Where the target would leave more
// than 8 blocks per range, the split count between those two bounds is the one
// that puts the fewest blocks on the busiest CU (workgroups per CU, rounded
// up, x blocks per range; ties to fewer splits): the workgroups of a launch
// spread one per CU in turn, so a count whose last turn fills only part of the
// CUs leaves those CUs one range more.  27648x5120 (40 column blocks, 216
// blocks): 27 splits (5 workgroups of 8 blocks on some CUs) -> 18 (3 of 12),
// same box, us, M = 1 / 4 / 8 / 16: 26.3 / 32.6 / 33.1 / 40.5 -> 25.7 / 29.9 /
// 31.2 / 33.5 (24 splits, 4 of 9: 25.0 / 30.7 / 31.7 / 34.1); the 5120 ->
// 2 x 27648 group 5 -> 4 splits, M = 4, 46.9 -> 45.5; 14336x4096 keeps 14
// (12: 16.5 / 20.7 / 23.6 against 14.9 / 20.0 / 22.6 at M = 1 / 4 / 16).
// Shorter inputs may likewise go down to half the target, keeping their
// K-parts per column pair, where that leaves fewer blocks on the busiest CU
// (ties keep the larger count): 5120x5120 8 -> 6 splits (320 workgroups, 2 on
// some CUs -> 240, one per CU), same box, us, M = 1 / 4 / 16: 10.14 / 13.21 /
// 16.04 -> 9.64 / 12.03 / 15.06.  4096x6144 keeps 8 (5 would change its K-parts
// and measured 9.52 against 9.31) and 5120x7168 keeps 8 (9: 11.19 / 14.69 /
// 18.04 against 11.33 / 14.37 / 17.82).
// Measured on MI355X (us, M = 1 / 4,
// same box): 4096x14336 4 splits 14.10 / 17.68, 8 13.72 / 17.41; 2048x1536
// 4: 7.57 / 9.98, 8: 6.59 / 8.50, 16: 7.32 / 9.83; 4096x6144 4: 11.41, 8:
// 9.41, 16: 11.05; 4096x4096 8: 8.63, 16: 9.62; 14336x4096 14: 14.97, 20:
// 15.28, 28: 16.25; 5120x7168 8: 11.24 / 14.26, 10: 11.35 / 15.56.
// Launches that would hold at most 1.25 waves per SIMD take 2 K-parts per
// column pair instead (two waves per pair meet in LDS: the same splits, twice
// the waves).  Same box, us, KW 1 -> 2 (M = 1 / 2 / 4 / 16): 4096x4096 (1024
// waves) 8.42 / 10.04 / 11.32 / 15.35 -> 8.21 / 9.64 / 10.16 / 14.27;
// 4096x1792 8.12 / 9.77 / 11.20 / 14.73 -> 7.89 / 9.32 / 9.98 / 13.53;
// 5120x5120 (1280) 10.45 / 12.58 / 13.58 / 17.8 -> 10.26 / 11.98 / 13.47 /
// 16.9; 2048x1536 6.50 -> 6.51; above the bound it loses at M = 1: 4096x6144
// (1536) 9.32 -> 9.62, 4096x10240 11.25 -> 12.43, 2048x12288 9.24 -> 9.56.
// Up to 2 waves per SIMD, ranges of at least 5 blocks (10 steps, 5 per wave
// after the split) take 2 K-parts as well: 5120x7168 (1792 waves, 5 blocks)
// 11.25 / 14.28 / 17.79 -> 10.92 / 13.76 / 16.92 at M = 1 / 4 / 16, 14336x4096
// (1792, 8 blocks) 14.99 / 19.65 / 22.62 -> 15.09 / 18.81 / 22.36.
// K = 5, 6 and 7 always take 2 K-parts: their weight loop keeps one slice in
// flight per set (register budget) and the decode of a 16 % K != 0 width needs a
// window per state, so a lone wave per column pair waits on its loads; twice the
// waves cover that (same box, us, KW 1 -> 2, M = 1 / 4 / 16: 4096x14336 K5
// 23.3 / 26.3 / 31.4 -> 21.6 / 21.5 / 27.3, K6 25.6 / 28.6 / 33.3 -> 21.7 / 21.8
// / 28.4, K7 34.8 / 37.8 / 42.1 -> 26.2 / 25.4 / 31.4; 27648x5120 K5 51.6 / 57.0 /
// 61.0 -> 33.5 / 45.9 / 53.6, K6 60.5 / 66.7 / 70.2 -> 34.0 / 47.0 / 55.1;
// 5120x27648 K5 52.5 / 59.1 -> 36.7 / 41.8 at M = 1 / 4).  4 K-parts lose
// (4096x14336 K5 M = 1 29.3).  K = 3 (a window per state as well, two slices per
// set) gains only with ranges of 8 or more blocks: 27648x5120 (12) 30.3 / 35.9 ->
// 27.2 / 34.5 at M = 1 / 4, 5120x27648 (8) 29.4 / 36.6 -> 29.3 / 34.9, but
// 4096x14336 (4) 14.5 / 18.3 / 22.9 -> 18.1 / 20.0 / 24.3 at M = 1 / 4 / 16.
// K = 8 loses with 2 everywhere (4096x14336 M = 1 22.0 -> 27.7, 27648x5120 M = 4
// 48.1 -> 56.9), and K = 4 does outside the waves rule (27648x5120 M = 4 29.9 ->
// 35.1).
// EXL3_QMV_SPLITS and EXL3_QMV_KW override (tuning).
static int simd_count();
static void choose_qmv_shape(int in, int out, int k, int* splits_out, int* kw_out) {
  const int nb = in / 128, col_blocks = out / 128;
  const int min_splits = (nb + 11) / 12, even_splits = (nb + 7) / 8;
  int kw = 0;
  if (const char* env = getenv("EXL3_QMV_KW")) {
    int v = atoi(env);
    if (v == 1 || v == 2 || v == 4) kw = v;
  }
  const int target_wgs = 896;
  int s = (target_wgs + col_blocks - 1) / col_blocks;
  s = std::min(s, std::max(1, std::min(8, nb / 2)));
  const int64_t cus = std::max(1, simd_count() / 4);
  auto busiest = [&](int c) {  // blocks on the busiest CU
    return (((int64_t)col_blocks * c + cus - 1) / cus) * ((nb + c - 1) / c);
  };
  auto k_parts = [&](int c) {
    if ((k >= 5 && k <= 7) || (k == 3 && (nb + c - 1) / c >= 8)) return 2;
    const int64_t waves = (int64_t)col_blocks * c * 4, simds = simd_count();
    return 4 * waves <= 5 * simds || (waves <= 2 * simds && (nb + c - 1) / c >= 5) ? 2 : 1;
  };
  if (s < even_splits) {
    int best = even_splits;
    int64_t best_cost = INT64_MAX;
    for (int c = std::max(s, min_splits); c <= even_splits; ++c) {
      const int64_t cost = busiest(c);
      if (cost < best_cost) {
        best_cost = cost;
        best = c;
      }
    }
    s = best;
  } else {
    // down to half the target, at the same K-parts per column pair: a count
    // whose workgroups spread more evenly over the CUs (ties keep the larger)
    int best = s;
    int64_t best_cost = busiest(s);
    for (int c = s - 1; c >= std::max(even_splits, (s + 1) / 2); --c) {
      if (k_parts(c) != k_parts(s)) continue;
      const int64_t cost = busiest(c);
      if (cost < best_cost) {
        best_cost = cost;
        best = c;
      }
    }
    s = best;
  }
  if (const char* env = getenv("EXL3_QMV_SPLITS")) {  // tuning: any split count that
    int v = atoi(env);                                 // keeps xhat within its LDS bound
    if (v >= 1) s = std::max(v, min_splits);
  }
  s = std::max(1, std::min(s, nb));
  if (kw == 0) kw = k_parts(s);
  *splits_out = s;
  *kw_out = kw;
}

// QMM launch shape: rows per workgroup 64*MB and global K-splits.  One
// workgroup fills a CU, so a launch runs in rounds of 256 workgroups, each
// round taking (K-steps per split) x (step time of that MB).  Step times
// fitted on MI355X with every CU busy: MB=1 660 ns, MB=2 750 ns, MB=4 1250 ns
// (per 64 input rows); a split adds its f32 partials (64*MB rows x 128 columns
// per tile, padded), written and read back through 16-byte coherent accesses
// at ~0.7 ns per KB.  Splits are only used while the output tiles alone fill
// at most 256 workgroups, so at most 256 tile counters are ever needed.
// Fitted to a sweep of MB {1,2,4} x splits {1,2,3,4,6,8} over 4096x14336 M
// {128, 512}, 14336x4096 M {128, 256, 512, 2048}, 27648x5120 and 5120x27648
// at M=128 and 4096x4096 at M=512; the partials' price refitted (1.0 -> 0.7 ns
// per KB) after the last arriver's loads went out 16 at a time, when a second
// sweep (14336x4096 M {128, 256, 512}, 27648x5120, 4096x14336 and 5120x27648
// at M=128, 4096x4096 at M=512) found the chosen shape fastest everywhere but
// 14336x4096 M=512 (MB=2, 2 splits 99.5 us against 93.7 for MB=4, 4 splits),
// which every price from 0.5 to 0.8 picks.
// EXL3_QMM_MB and EXL3_QMM_SPLITS override.
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
  QmmShape best{4, (int)((rows + 255) / 256), 1};
  double best_cost = 1e300;
  for (int mb : {4, 2, 1}) {
    if (force_mb && mb != force_mb) continue;
    const double step_ns = mb == 4 ? 1250.0 : mb == 2 ? 750.0 : 660.0;
    const int64_t mt = (rows + 64 * mb - 1) / (64 * mb);
    const int64_t base = mt * col_blocks;
    for (int splits : {1, 2, 3, 4, 6, 8}) {
      int s = force_splits ? force_splits : splits;
      s = std::max(1, std::min(s, std::max(1, nq / 4)));
      if (s > 1 && base > kTileCounters) s = 1;
      const int64_t rounds = (base * s + 255) / 256;
      double cost = (double)rounds * ((nq + s - 1) / s) * step_ns;
      if (s > 1) cost += 0.7 / 1024 * 4.0 * (double)s * mt * 64 * mb * out;
      if (cost < best_cost) {
        best_cost = cost;
        best = QmmShape{mb, (int)mt, s};
      }
      if (force_splits) break;
    }
  }
  return best;
}

// Split-K partials of a QMM launch: per split and output tile, the f32
// accumulators of its 64*MB rows x 128 columns in fragment order.
static size_t qmm_partial_bytes(const QmmShape& sh, int out) {
  if (sh.splits <= 1) return 0;
  return sizeof(float) * (size_t)sh.splits * sh.mtiles * (out / 128) * 64 * sh.mb * 128;
}

// Workspace: the first kWorkspaceCounterBytes hold split-K counters that are
// zero between calls (every call leaves them zero, so one workspace serves
// every entry point in any order).  The rest is per-call scratch: QMV
// partials, or QMM xhat rows (one set per member) and partials.
static constexpr int kCounterWords = (int)(kWorkspaceCounterBytes / sizeof(uint32_t));

// A launch over 1..kMaxMembers projections sharing one input.
struct Group {
  const exl3_linear* parts[kMaxMembers];
  int count, in, total_out, k, cb;
};

static int make_group(const exl3_linear* const* parts, int count, Group& g) {
  if (!parts || count < 1) return fail(EXL3_EINVAL, "empty EXL3 group");
  if (count > kMaxMembers)
    return fail(EXL3_EUNSUPPORTED, "EXL3 groups of more than %d projections are not supported",
                kMaxMembers);
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    if (!parts[i]) return fail(EXL3_EINVAL, "null EXL3 group member %d", i);
    if (parts[i]->in != parts[0]->in || parts[i]->k != parts[0]->k ||
        parts[i]->cb != parts[0]->cb)
      return fail(EXL3_EINVAL, "EXL3 group members need the same input width, K and codebook");
    g.parts[i] = parts[i];
    total += parts[i]->out;
  }
  if (total > INT32_MAX || total / 128 > kCounterWords)
    return fail(EXL3_EUNSUPPORTED, "EXL3 group too wide: %lld columns", (long long)total);
  g.count = count;
  g.in = parts[0]->in;
  g.total_out = (int)total;
  g.k = parts[0]->k;
  g.cb = parts[0]->cb;
  return EXL3_OK;
}

static void group_qmv_shape(const Group& g, int* splits, int* kw) {
  if (g.count == 1) {
    *splits = g.parts[0]->qmv_splits;
    *kw = g.parts[0]->qmv_kw;
  } else {
    choose_qmv_shape(g.in, g.total_out, g.k, splits, kw);
  }
}

// The QMV computes xhat in every workgroup for its K-range (rows x blocks
// prologue jobs, a few hundred cycles each); once that reaches 64 jobs per
// workgroup, one separate prologue launch (~3.5 us) is cheaper.  Measured on
// MI355X: 4096x14336 M=8 22.5 vs 24.1 us, M=4 21.2 vs 19.8 us; 4096x4096 M=16
// 20.7 vs 19.2 us.  Every column block repeats the jobs of its K-range, so a
// launch computes rows x blocks x column blocks of them in all: multi-row
// launches past kProloguePerLaunch jobs also take the separate launch (the
// 4-row gate/up of a 5120 -> 2 x 27648 group repeats 69 k jobs, ~10 us of VALU
// issue).  EXL3_QMV_PROLOGUE_JOBS overrides that total (0: off; tuning).
static constexpr int64_t kProloguePerLaunch = 20480;
static bool qmv_separate_prologue(const Group& g, int64_t rows, int splits) {
  static const int64_t per_launch = [] {
    const char* env = getenv("EXL3_QMV_PROLOGUE_JOBS");
    return env ? (int64_t)atoll(env) : kProloguePerLaunch;
  }();
  const int nb = g.in / 128;
  const int blocks = (nb + splits - 1) / splits;  // the largest K-range of a split
  if (rows * blocks >= 64) return true;
  return rows > 1 && per_launch > 0 && rows * nb * (int64_t)(g.total_out / 128) >= per_launch;
}

// Multi-row QMVs of at least this many rows (one K-part per column pair)
// exchange their split-K partials in fragment order: 8 KB slabs per split and
// column block written and read with 16-byte coherent accesses, instead of
// 4-byte row-major ones.  EXL3_QMV_FRAG_ROWS overrides it (tuning).
static bool qmv_fragment_exchange(int64_t rows, int kw) {
  static const int from = [] {
    const char* env = getenv("EXL3_QMV_FRAG_ROWS");
    return env ? atoi(env) : 8;
  }();
  return kw == 1 && rows >= from;
}

// Scratch bytes (after the counter region) of one group launch.
static size_t group_scratch_bytes(const Group& g, int64_t rows) {
  if (rows <= kQmvMaxRows) {
    int splits, kw;
    group_qmv_shape(g, &splits, &kw);
    const size_t xhat = qmv_separate_prologue(g, rows, splits)
                            ? g.count * align_up(sizeof(uint16_t) * (size_t)rows * g.in)
                            : 0;
    // partials: 8 KB fragment slabs per split and column block, or one
    // row-major f32 row per split and row
    const size_t partials = qmv_fragment_exchange(rows, kw)
                                ? (size_t)splits * (g.total_out / 128) * 8192
                                : sizeof(float) * (size_t)splits * rows * g.total_out;
    return xhat + align_up(partials);
  }
  const QmmShape sh = choose_qmm_shape(g.in, g.total_out, rows);
  const size_t partials = qmm_partial_bytes(sh, g.total_out);
  return (size_t)g.count * align_up(sizeof(uint16_t) * (size_t)rows * g.in) + align_up(partials);
}

static int check_rows(const Group& g, int64_t rows) {
  if (rows < 1) return fail(EXL3_EINVAL, "EXL3 linear input cannot be empty");
  if (rows > (int64_t)INT32_MAX / std::max(g.in, g.total_out))
    return fail(EXL3_EINVAL, "EXL3 linear input too large: %lld rows", (long long)rows);
  return EXL3_OK;
}

static Member member_of(const exl3_linear* h, void* y, int cblk0, int x_type) {
  Member m;
  m.trellis = (const uint32_t*)h->trellis;
  m.suh = h->suh;
  m.xhat = nullptr;
  m.svh = h->svh;
  m.bias = h->bias;
  m.y = y;
  m.out = h->out;
  m.cblk0 = cblk0;
  m.y_dtype = result_dtype(x_type, h->bias != nullptr);
  return m;
}

// SIMDs of the current device (4 per CU), cached per device.
static int simd_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = 4 * cus;
  }
  return cached[dev];
}

// One QMV launch (rows <= 16) over the group; `glu` for a (gate, up) pair.
// `given_xhat`: the single member's xhat, already computed (no prologue here).
static int run_group_qmv(const Group& g, const void* x, int x_type, int64_t rows,
                         void* const* ys, uint32_t* counters, char* scratch, const Glu& glu,
                         hipStream_t stream, const uint16_t* given_xhat = nullptr) {
  if (int rc = launch_gate("EXL3 QMV launch")) return rc;
  QmvParams p{};
  int cblk0 = 0;
  for (int i = 0; i < g.count; ++i) {
    p.mem[i] = member_of(g.parts[i], ys[i], cblk0, x_type);
    cblk0 += g.parts[i]->out / 128;
  }
  int kw;
  group_qmv_shape(g, &p.splits, &kw);
  if (given_xhat) {
    if (g.count != 1) return fail(EXL3_EINVAL, "a precomputed xhat serves one projection");
    p.mem[0].xhat = given_xhat;
  } else if (qmv_separate_prologue(g, rows, p.splits)) {
    const size_t xbytes = align_up(sizeof(uint16_t) * (size_t)rows * g.in);
    PrologueParams pp{};
    pp.x = x;
    pp.x_dtype = x_type;
    pp.in = g.in;
    pp.rows = (int)rows;
    for (int i = 0; i < g.count; ++i) {
      pp.suh[i] = g.parts[i]->suh;
      pp.xhat[i] = (uint16_t*)(scratch + i * xbytes);
      p.mem[i].xhat = pp.xhat[i];
    }
    launch_prologue(pp, g.count, stream);
    if (int rc = check_launch("EXL3 prologue launch")) return rc;
    scratch += g.count * xbytes;
  }
  p.members = g.count;
  p.x = x;
  p.partials = (float*)scratch;
  p.counters = counters;
  p.in = g.in;
  p.total_out = g.total_out;
  p.M = (int)rows;
  p.x_dtype = x_type;
  p.glu = glu;
  const int64_t waves = (int64_t)(g.total_out / 128) * p.splits * 4 * kw;
  p.prio_ramp = waves > simd_count();
  const int nb = g.in / 128;
  int max_blocks = 0;
  for (int s = 0; s < p.splits; ++s)
    max_blocks = std::max(max_blocks, (s + 1) * nb / p.splits - s * nb / p.splits);
  size_t lds = sizeof(uint16_t) * (size_t)rows * max_blocks * 128;
  const int kwi = kw == 4 ? 2 : kw == 2 ? 1 : 0;
  const bool single = rows == 1 && kw == 1 && !glu.on && !p.mem[0].xhat;
  const bool frag = !single && qmv_fragment_exchange(rows, kw);
  // the fragment exchange sums a column block's rows (f32, both members of a
  // SwiGLU pair) in the activation buffer's LDS
  if (frag) lds = std::max(lds, sizeof(float) * 128 * (size_t)rows * (glu.on ? 2 : 1));
  static const int shallow_env = [] {  // EXL3_QMV_SHALLOW=0/1 overrides (tuning)
    const char* env = getenv("EXL3_QMV_SHALLOW");
    return env ? atoi(env) : -1;
  }();
  // One slice per prefetch set (and the first step decoded under the
  // prologue) from 3 waves per SIMD; multi-row launches only with K-ranges of
  // up to 4 blocks (same box, us, two-deep -> shallow: 4096x14336 M=2/4/8/16
  // 15.28/17.11/19.47/20.71 -> 15.09/16.90/18.74/20.45, 4096x28672 M=4 26.27
  // -> 25.51, 2048x12288 M=4 11.32 -> 11.21; 8-block ranges lose: 5120x27648
  // M=4 31.98 -> 32.43, 5120x55296 M=4 49.28 -> 49.74, 27648x5120 M=4 36.04 ->
  // 36.69, while one row gains there too: 5120x27648 25.95 -> 25.72).
  const bool shallow =
      shallow_env >= 0 ? shallow_env > 0
                       : waves >= 3 * (int64_t)simd_count() && (single || max_blocks <= 4);
  // one row, 2 K-parts per pair: the single-row kernel in its shallow form
  const bool single2 = rows == 1 && kw == 2 && !glu.on && !p.mem[0].xhat;
  const QmvFn fn = single2 ? kQmvSingle2[g.k - 1][g.cb]
                   : single ? (shallow ? kQmvSingleShallow : kQmvSingle)[g.k - 1][g.cb]
                   : frag ? (shallow ? kQmvFragShallow : kQmvFrag)[g.k - 1][g.cb]
                   : kw == 1 && shallow ? kQmvShallow[g.k - 1][g.cb]
                                        : kQmv[kwi][g.k - 1][g.cb];
  fn(p, dim3(g.total_out / 128, p.splits), lds, stream);
  return check_launch("EXL3 QMV launch");
}

// Prologue (one launch for all members) and one QMM launch over the group.
// xhats: per member, null to run the prologue into the scratch.
static int run_group_qmm(const Group& g, const void* x, int x_type, int64_t rows,
                         void* const* ys, uint32_t* counters, char* scratch,
                         const uint16_t* given_xhat, hipStream_t stream) {
  if (int rc = launch_gate("EXL3 QMM launch")) return rc;
  const size_t xbytes = align_up(sizeof(uint16_t) * (size_t)rows * g.in);
  QmmParams q{};
  if (!given_xhat) {
    PrologueParams pp{};
    pp.x = x;
    pp.x_dtype = x_type;
    pp.in = g.in;
    pp.rows = (int)rows;
    for (int i = 0; i < g.count; ++i) {
      pp.suh[i] = g.parts[i]->suh;
      pp.xhat[i] = (uint16_t*)(scratch + i * xbytes);
    }
    launch_prologue(pp, g.count, stream);
    if (int rc = check_launch("EXL3 prologue launch")) return rc;
  }
  int cblk0 = 0;
  for (int i = 0; i < g.count; ++i) {
    q.mem[i] = member_of(g.parts[i], ys[i], cblk0, x_type);
    q.mem[i].xhat = given_xhat ? given_xhat : (const uint16_t*)(scratch + i * xbytes);
    cblk0 += g.parts[i]->out / 128;
  }
  const QmmShape sh = choose_qmm_shape(g.in, g.total_out, rows);
  q.members = g.count;
  q.partials = (float*)(scratch + (given_xhat ? 0 : g.count * xbytes));
  q.counters = counters;
  q.in = g.in;
  q.total_out = g.total_out;
  q.M = (int)rows;
  q.x_dtype = x_type;
  q.col_blocks = g.total_out / 128;
  q.mtiles = sh.mtiles;
  q.splits = sh.splits;
  const int mbi = sh.mb == 4 ? 2 : sh.mb == 2 ? 1 : 0;
  const int64_t wgs = (int64_t)sh.mtiles * q.col_blocks * sh.splits;
  if (wgs > INT32_MAX) return fail(EXL3_EINVAL, "EXL3 QMM grid too large");
  kQmm[mbi][g.k - 1][g.cb](q, dim3((unsigned)wgs), stream);
  return check_launch("EXL3 QMM launch");
}

static int group_forward(const Group& g, const void* x, int x_type, int64_t rows,
                         void* const* ys, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!x) return fail(EXL3_EINVAL, "null activation pointer");
  for (int i = 0; i < g.count; ++i)
    if (!ys[i]) return fail(EXL3_EINVAL, "null activation pointer");
  if (!valid_dtype(x_type)) return fail(EXL3_EINVAL, "unsupported activation dtype code %d", x_type);
  if (int rc = check_rows(g, rows)) return rc;
  const size_t need = kWorkspaceCounterBytes + group_scratch_bytes(g, rows);
  if (!ws || ws_bytes < need)
    return fail(EXL3_EINVAL, "workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
  uint32_t* counters = (uint32_t*)ws;
  char* scratch = (char*)ws + kWorkspaceCounterBytes;
  const Glu none{};
  if (rows <= kQmvMaxRows) return run_group_qmv(g, x, x_type, rows, ys, counters, scratch, none, stream);
  return run_group_qmm(g, x, x_type, rows, ys, counters, scratch, nullptr, stream);
}

// ---------------------------------------------------------------------------
// SwiGLU MLP: y = down(swiglu(gate(x), up(x))), f16 activations.
// rows <= 16: one (gate, up) QMV launch whose epilogue applies the SwiGLU
// (the last workgroup of a column block pair holds both partial sums), then
// the down QMV (its prologue fused as for any linear): 2 launches.
// rows > 16: the (gate, up) group (prologue + QMM), one kernel applying the
// SwiGLU and the down projection's prologue, then the down QMM on that xhat:
// 4 launches instead of 6, and the activation never round-trips HBM.
// ---------------------------------------------------------------------------
static int mlp_check(const exl3_linear* gate, const exl3_linear* up, const exl3_linear* down) {
  if (!gate || !up || !down) return fail(EXL3_EINVAL, "null EXL3 MLP projection");
  if (gate->in != up->in || gate->out != up->out || gate->k != up->k || gate->cb != up->cb)
    return fail(EXL3_EINVAL, "incompatible grouped projections");
  if (down->in != gate->out)
    return fail(EXL3_EINVAL, "EXL3 MLP down projection expects %d inputs, gate/up give %d",
                down->in, gate->out);
  return EXL3_OK;
}

static size_t mlp_ws_bytes(const exl3_linear* gate, const exl3_linear* up,
                           const exl3_linear* down, int64_t rows) {
  const exl3_linear* gu[2] = {gate, up};
  Group g;
  if (make_group(gu, 2, g)) return 0;
  const size_t act = align_up(sizeof(uint16_t) * (size_t)rows * gate->out);
  size_t need;
  if (rows <= kQmvMaxRows) {
    Group d;
    if (make_group(&down, 1, d)) return 0;
    need = act + std::max(group_scratch_bytes(g, rows), group_scratch_bytes(d, rows));
  } else {
    const QmmShape sh = choose_qmm_shape(down->in, down->out, rows);
    const size_t stage2 = align_up(qmm_partial_bytes(sh, down->out));
    // down xhat + gate and up outputs
    need = 3 * act + std::max(group_scratch_bytes(g, rows), stage2);
  }
  return kWorkspaceCounterBytes + need;
}

static int mlp_forward(const exl3_linear* gate, const exl3_linear* up, const exl3_linear* down,
                       const void* x, int x_type, int64_t rows, void* y, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
  if (int rc = mlp_check(gate, up, down)) return rc;
  if (!x || !y) return fail(EXL3_EINVAL, "null activation pointer");
  if (x_type != EXL3_F16)
    return fail(EXL3_EUNSUPPORTED, "the fused SwiGLU MLP takes f16 activations (dtype %d)",
                x_type);
  const exl3_linear* gu[2] = {gate, up};
  Group g, d;
  if (int rc = make_group(gu, 2, g)) return rc;
  if (int rc = make_group(&down, 1, d)) return rc;
  if (int rc = check_rows(g, rows)) return rc;
  if (int rc = check_rows(d, rows)) return rc;
  const size_t need = mlp_ws_bytes(gate, up, down, rows);
  if (!ws || ws_bytes < need)
    return fail(EXL3_EINVAL, "workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
  uint32_t* counters = (uint32_t*)ws;
  char* base = (char*)ws + kWorkspaceCounterBytes;
  uint16_t* act = (uint16_t*)base;  // the activation (QMV) or the down xhat (QMM)
  const size_t act_bytes = align_up(sizeof(uint16_t) * (size_t)rows * gate->out);
  void* dy[1] = {y};
  if (rows <= kQmvMaxRows) {
    Glu glu{};
    glu.on = 1;
    glu.out = act;
    // Where the down projection would run its prologue as a launch of its
    // own, the gate/up epilogue applies it to each finished 128-block instead
    // (f16(a * suh), the staged H128, f16(* 1/sqrt(128))) and down reads that
    // xhat: one launch fewer per MLP.
    int dsplits, dkw;
    group_qmv_shape(d, &dsplits, &dkw);
    const bool down_xhat = qmv_separate_prologue(d, rows, dsplits);
    if (down_xhat) glu.down_suh = down->suh;
    void* gu_y[2] = {nullptr, nullptr};  // not written: the edge consumes the partials
    if (int rc = run_group_qmv(g, x, EXL3_F16, rows, gu_y, counters, base + act_bytes, glu, stream))
      return rc;
    return run_group_qmv(d, act, EXL3_F16, rows, dy, counters, base + act_bytes, Glu{}, stream,
                         down_xhat ? act : nullptr);
  }
  void* gu_y[2] = {base + act_bytes, base + 2 * act_bytes};
  char* scratch = base + 3 * act_bytes;
  if (int rc = run_group_qmm(g, x, EXL3_F16, rows, gu_y, counters, scratch, nullptr, stream))
    return rc;
  if (int rc = launch_gate("SwiGLU prepare launch")) return rc;
  launch_swiglu_prepare((const uint16_t*)gu_y[0], (const uint16_t*)gu_y[1], down->suh, gate->out,
                        (int)rows, act, stream);
  if (int rc = check_launch("SwiGLU prepare launch")) return rc;
  return run_group_qmm(d, nullptr, EXL3_F16, rows, dy, counters, scratch, act, stream);
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
  // The kernels address a trellis with 32-bit byte offsets from a base inside it.
  const int64_t trellis_bytes = (int64_t)in * out / 8 * k;
  if (trellis_bytes >= ((int64_t)1 << 32))
    return fail(EXL3_EINVAL, "EXL3 trellis of %lld bytes exceeds the 4 GiB limit",
                (long long)trellis_bytes);
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
  choose_qmv_shape(in, out, k, &h->qmv_splits, &h->qmv_kw);
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
  Group g;
  if (!h || rows < 1 || make_group(&h, 1, g)) return 0;
  return kWorkspaceCounterBytes + group_scratch_bytes(g, rows);
}

size_t exl3_group_workspace_bytes(const exl3_linear* const* parts, int32_t count, int64_t rows) {
  Group g;
  if (rows < 1 || make_group(parts, count, g)) return 0;
  return kWorkspaceCounterBytes + group_scratch_bytes(g, rows);
}

size_t exl3_mlp_workspace_bytes(const exl3_linear* gate, const exl3_linear* up,
                                const exl3_linear* down, int64_t rows) {
  if (rows < 1 || mlp_check(gate, up, down)) return 0;
  return mlp_ws_bytes(gate, up, down, rows);
}

int exl3_workspace_init(void* workspace, size_t bytes, void* stream) {
  if (!workspace || bytes % 4) return fail(EXL3_EINVAL, "workspace must be non-null, 4-byte sized");
  const size_t words = bytes / 4;
  if (words == 0) return EXL3_OK;
  launch_fill_zero((uint32_t*)workspace, words, (hipStream_t)stream);
  return check_launch("workspace init");
}

int32_t exl3_linear_output_dtype(const exl3_linear* h, int32_t x_type) {
  if (!h || !valid_dtype(x_type)) return -1;
  return result_dtype(x_type, h->bias != nullptr);
}

int exl3_linear_forward(const exl3_linear* h, const void* x, int32_t x_type, int64_t rows, void* y,
                        int32_t y_type, void* workspace, size_t workspace_bytes, void* stream) {
  if (!h) return fail(EXL3_EINVAL, "null EXL3 linear handle");
  if (!valid_dtype(x_type)) return fail(EXL3_EINVAL, "unsupported activation dtype code %d", x_type);
  const int want = result_dtype(x_type, h->bias != nullptr);
  if (y_type != want)
    return fail(EXL3_EINVAL,
                "EXL3 output dtype %d differs from the projection's result dtype %d (the input "
                "dtype, promoted with the f16 bias)",
                y_type, want);
  Group g;
  if (int rc = make_group(&h, 1, g)) return rc;
  return group_forward(g, x, x_type, rows, &y, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t exl3_linear_noalloc_max_bytes(void) { return kNoAllocBytes; }

int exl3_linear_forward_noalloc(const exl3_linear* h, const void* x, int32_t x_type, int64_t rows,
                                void* y, int32_t y_type, void* stream) {
  if (!h) return fail(EXL3_EINVAL, "null EXL3 linear handle");
  if (!valid_dtype(x_type)) return fail(EXL3_EINVAL, "unsupported activation dtype code %d", x_type);
  Group g;
  if (int rc = make_group(&h, 1, g)) return rc;
  if (int rc = check_rows(g, rows)) return rc;
  const size_t need = kWorkspaceCounterBytes + group_scratch_bytes(g, rows);
  if (need > kNoAllocBytes)
    return fail(EXL3_EUNSUPPORTED,
                "allocation-free EXL3 forward of %lld rows needs %zu bytes of workspace, more "
                "than its fixed %zu; use exl3_linear_forward with a caller workspace",
                (long long)rows, need, kNoAllocBytes);
  void* ws = nullptr;
  if (int rc = noalloc_scratch((hipStream_t)stream, &ws)) return rc;
  return exl3_linear_forward(h, x, x_type, rows, y, y_type, ws, kNoAllocBytes, stream);
}

int exl3_group_forward(const exl3_linear* const* parts, int32_t count, const void* x,
                       int32_t x_type, int64_t rows, void* const* ys, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (!ys) return fail(EXL3_EINVAL, "empty EXL3 group");
  Group g;
  if (int rc = make_group(parts, count, g)) return rc;
  return group_forward(g, x, x_type, rows, ys, workspace, workspace_bytes, (hipStream_t)stream);
}

int exl3_mlp_forward(const exl3_linear* gate, const exl3_linear* up, const exl3_linear* down,
                     const uint16_t* x, int64_t rows, uint16_t* y, void* workspace,
                     size_t workspace_bytes, void* stream) {
  return mlp_forward(gate, up, down, x, EXL3_F16, rows, y, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

int exl3_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t count,
                void* stream) {
  if (count < 0) return fail(EXL3_EINVAL, "negative element count");
  if (count == 0) return EXL3_OK;
  if (!gate || !up || !out) return fail(EXL3_EINVAL, "null SwiGLU buffer");
  if (int rc = launch_gate("SwiGLU launch")) return rc;
  launch_glu(gate, up, out, count, false, (hipStream_t)stream);
  return check_launch("SwiGLU launch");
}

int exl3_geglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t count,
               void* stream) {
  if (count < 0) return fail(EXL3_EINVAL, "negative element count");
  if (count == 0) return EXL3_OK;
  if (!gate || !up || !out) return fail(EXL3_EINVAL, "null GEGLU buffer");
  if (int rc = launch_gate("GEGLU launch")) return rc;
  launch_glu(gate, up, out, count, true, (hipStream_t)stream);
  return check_launch("GEGLU launch");
}

int exl3_prepare128(const uint16_t* x, int64_t elements, int32_t width, const uint16_t* scales,
                    int64_t scale_count, uint16_t* out, void* stream) {
  // prepare128_blocks (contracts.rs:2146-2159): u32 extents, complete rows of
  // a 128-aligned width, one scale per column or per element
  if (elements < 0 || elements > (int64_t)UINT32_MAX || width <= 0 || width % 128 ||
      elements % width || (scale_count != width && scale_count != elements))
    return fail(EXL3_EINVAL, "expected complete 128-aligned rows and column or element scales");
  if (elements == 0) return EXL3_OK;
  if (!x || !scales || !out) return fail(EXL3_EINVAL, "null prepare128 buffer");
  if (int rc = launch_gate("EXL3 prepare128 launch")) return rc;
  PrologueParams pp{};
  pp.x = x;
  pp.x_dtype = EXL3_F16;
  pp.in = width;
  pp.rows = (int)(elements / width);
  pp.suh[0] = scales;
  pp.xhat[0] = out;
  pp.suh_stride = scale_count == elements ? (size_t)width : 0;
  launch_prologue(pp, 1, (hipStream_t)stream);
  return check_launch("EXL3 prepare128 launch");
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

int exl3_pack_tiles(const uint16_t* states, int64_t tiles, int32_t k, uint16_t* packed,
                    void* stream) {
  if (k < 1 || k > 8) return fail(EXL3_EINVAL, "K must be in 1..=8, got %d", k);
  if (tiles < 0) return fail(EXL3_EINVAL, "negative tile count");
  if (tiles == 0) return EXL3_OK;
  if (!states || !packed) return fail(EXL3_EINVAL, "null pack buffer");
  if ((tiles * 16 * k + 255) / 256 > INT32_MAX) return fail(EXL3_EINVAL, "too many tiles");
  launch_pack_tiles(states, tiles, k, packed, (hipStream_t)stream);
  return check_launch("EXL3 pack launch");
}

int exl3_codewords(const uint16_t* states, int64_t count, int32_t cb, uint16_t* values,
                   void* stream) {
  if (cb < 0 || cb > 2) return fail(EXL3_EINVAL, "invalid EXL3 codebook %d", cb);
  if (count < 0) return fail(EXL3_EINVAL, "negative element count");
  if (count == 0) return EXL3_OK;
  if (!states || !values) return fail(EXL3_EINVAL, "null codeword buffer");
  if ((count + 255) / 256 > INT32_MAX) return fail(EXL3_EINVAL, "too many states");
  launch_codewords(states, count, cb, values, (hipStream_t)stream);
  return check_launch("EXL3 codeword launch");
}

size_t exl3_qmv_inner_workspace_bytes(int32_t rows, int32_t cols) {
  if (rows <= 0 || cols <= 0 || rows % 16 || cols % 16) return 0;
  return align_up(sizeof(uint16_t) * (size_t)rows * cols);
}

int exl3_qmv_inner(const uint16_t* packed, int32_t rows, int32_t cols, int32_t k, int32_t cb,
                   const uint16_t* x, uint16_t* y, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (k < 1 || k > 8) return fail(EXL3_EINVAL, "K must be in 1..=8, got %d", k);
  if (cb < 0 || cb > 2) return fail(EXL3_EINVAL, "invalid EXL3 codebook %d", cb);
  if (rows <= 0 || cols <= 0 || rows % 16 || cols % 16)
    return fail(EXL3_EINVAL, "expected positive 16-aligned dimensions");
  if (!packed || !x || !y) return fail(EXL3_EINVAL, "null QMV buffer");
  const size_t need = exl3_qmv_inner_workspace_bytes(rows, cols);
  if (!workspace || workspace_bytes < need)
    return fail(EXL3_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes,
                need);
  const int64_t tiles = (int64_t)(rows / 16) * (cols / 16);
  int rc = exl3_decode_tiles(packed, tiles, k, cb, nullptr, (uint16_t*)workspace, stream);
  if (rc) return rc;
  launch_qmv_inner((const uint16_t*)workspace, x, rows, cols, y, (hipStream_t)stream);
  return check_launch("EXL3 inner QMV launch");
}

}  // extern "C"

