// The mapped expert QMV, expert_mapped (native/src/linear.rs:2817-2852, with
// expert_mapped_layout :3054-3336 for a route-major bank): every row of x has
// its own weight columns, chosen by its route's expert in a bank of tiles.
//
//   row r = route * P + p,  P = projections per route;
//   tile columns of row r:  selected[route] * OT + p * stride + t,  t < OT = out/16;
//   xhat_r = f16(H128(f16(f16(x_r) * suh_r)) / sqrt 128)  (per-row input scales);
//   yhat_r = xhat_r . W[:, columns of r]  (f32);
//   raw:  y_r = yhat_r (f32);  else  y_r = f16(H128(f16(yhat_r)) / sqrt 128) * svh_r,
//         cast to x's dtype (the linear's output epilogue with per-row scales).
//
// Three launches: the input prologue (per-row scales) into the workspace,
// mapped_kernel (one workgroup per (row, 128-column block, K-range), the QMV's
// per-wave decode loop with the row's xhat read from L2), and mapped_finish
// (split sums in split order, then the epilogue or the raw store).  The split
// count depends on the input width only, so a row's result does not depend on
// the other rows of the call.  Rows whose tile columns fall outside the bank
// produce zeros instead of reading past it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/exl3_hip.h"
#include "exl3_launch.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {

struct MappedParams {
  const uint32_t* trellis;   // [in/16][bank_tiles][8K] u32
  const uint16_t* xhat;      // [rows][in] f16
  const uint32_t* selected;  // [routes]
  float* partials;           // [splits][rows][out] f32
  int in, out, bank_tiles, projections, stride_tiles, rows, splits;
};

// Tile-column base of row `row`, or -1 when its columns leave the bank.
__device__ __forceinline__ int64_t mapped_base(const MappedParams& p, int row) {
  const int route = row / p.projections, proj = row - route * p.projections;
  const int64_t ot = p.out >> 4;
  const int64_t base = (int64_t)p.selected[route] * ot + (int64_t)proj * p.stride_tiles;
  return base + ot <= p.bank_tiles ? base : -1;
}

// grid (rows * out/128, splits), 256 threads: wave w decodes tile columns
// 2w, 2w+1 of the 128-column block over the split's 64-input steps, all 16
// MFMA rows reading the row's xhat (row 0 of the product is stored).
template <int K, int CB>
__global__ __launch_bounds__(256) void mapped_kernel(MappedParams p) {
  const int lane = threadIdx.x & 63, pair = threadIdx.x >> 6;
  const int col_blocks = p.out >> 7;
  const int row = blockIdx.x / col_blocks, cblk = blockIdx.x - row * col_blocks;
  const int split = blockIdx.y;
  const int64_t base = mapped_base(p, row);
  const int nq_all = p.in >> 6;
  const int qa = split * nq_all / p.splits, nq = (split + 1) * nq_all / p.splits - qa;
  const int g = lane >> 4, hsel = (lane >> 3) & 1, j = lane & 7;
  const int64_t tcol = (base < 0 ? 0 : base) + cblk * 8 + pair * 2 + hsel;
  const uint32_t* tp =
      p.trellis + ((size_t)(4 * qa + g) * p.bank_tiles + tcol) * (8 * K) + (size_t)j * K;
  const size_t qstride = (size_t)4 * p.bank_tiles * 8 * K;
  const int prev_off = j == 0 ? 8 * K - 1 : -1;
  const _Float16* xrow = (const _Float16*)p.xhat + (size_t)row * p.in + 64 * qa + 16 * g;
  const int qlast = nq - 1;
  constexpr int D = kQmvDepth<K>;
  uint32_t setA[D][K + 1], setB[D][K + 1];
  float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  auto fetch = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      load_slice_prev<K>(tp + (size_t)min(qbase + d, qlast) * qstride, prev_off, set[d]);
  };
  auto compute = [&](uint32_t(&set)[D][K + 1], int qbase) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int q = qbase + d;
      if (q < nq) {
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
  // accumulator lane l < 16 holds row 0 at column 16 (2 pair + l / 8) + l % 8
  // (+ 8 for acc1)
  if (g == 0) {
    const int col = cblk * 128 + 16 * (pair * 2 + (lane >> 3)) + (lane & 7);
    float* part = p.partials + ((size_t)split * p.rows + row) * p.out;
    part[col] = base < 0 ? 0.f : acc0[0];
    part[col + 8] = base < 0 ? 0.f : acc1[0];
  }
}

// grid (rows * out/128), 64 threads: lane holds columns (lane, lane + 64) of a
// 128-column block; splits added in split order.
__global__ __launch_bounds__(64) void mapped_finish(const float* __restrict__ partials, int rows,
                                                    int out, int splits,
                                                    const uint16_t* __restrict__ svh, int raw,
                                                    int x_dtype, void* y) {
  const int col_blocks = out >> 7;
  const int row = blockIdx.x / col_blocks, cblk = blockIdx.x - row * col_blocks;
  const int lane = threadIdx.x;
  const size_t off = (size_t)row * out + cblk * 128;
  float v0 = 0.f, v1 = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float* ps = partials + (size_t)s * rows * out + off;
    v0 += ps[lane];
    v1 += ps[lane + 64];
  }
  if (raw) {
    ((float*)y)[off + lane] = v0;
    ((float*)y)[off + lane + 64] = v1;
    return;
  }
  finish_row128(v0, v1, lane, cblk * 128, svh + (size_t)row * out, nullptr, y, x_dtype, x_dtype,
                (size_t)row * out);
}

#define EXL3_MAPPED_INST(K, CB) template __global__ void mapped_kernel<K, CB>(MappedParams);
EXL3_INSTANTIATE(EXL3_MAPPED_INST)

}  // namespace exl3

using namespace exl3;

#ifndef __HIP_DEVICE_COMPILE__

namespace {
typedef void (*MappedFn)(MappedParams);
#define EXL3_MAPPED_ROW(K) {mapped_kernel<K, 0>, mapped_kernel<K, 1>, mapped_kernel<K, 2>}
const MappedFn kMapped[8][3] = {EXL3_MAPPED_ROW(1), EXL3_MAPPED_ROW(2), EXL3_MAPPED_ROW(3),
                                EXL3_MAPPED_ROW(4), EXL3_MAPPED_ROW(5), EXL3_MAPPED_ROW(6),
                                EXL3_MAPPED_ROW(7), EXL3_MAPPED_ROW(8)};

// K-ranges of at least 8 steps of 64 inputs, at most 8 (a function of the
// input width only: rows stay independent of each other).
int mapped_splits(int in) { return std::max(1, std::min(8, in / 64 / 8)); }

size_t align256(size_t v) { return (v + 255) / 256 * 256; }
}  // namespace

extern "C" size_t exl3_expert_mapped_workspace_bytes(int32_t in, int32_t out, int64_t rows) {
  if (in <= 0 || out <= 0 || rows <= 0) return 0;
  return kWorkspaceCounterBytes + align256((size_t)rows * in * 2) +
         align256((size_t)mapped_splits(in) * rows * out * 4);
}

extern "C" int exl3_expert_mapped(const uint16_t* trellis, int32_t in, int32_t bank_tiles,
                                  int32_t k, int32_t cb, const void* x, int32_t x_type,
                                  int64_t rows, const uint16_t* suh, const uint32_t* selected,
                                  int32_t routes, int32_t projections, int32_t out,
                                  int32_t stride_tiles, const uint16_t* svh, int32_t raw, void* y,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  // checks of expert_mapped_layout (linear.rs:3074-3127), in its order
  if (k < 1 || k > 8) return fail(EXL3_EINVAL, "K must be in 1..=8, got %d", k);
  if (k == 7) return fail(EXL3_EUNSUPPORTED, "mapped K=7 is not supported");
  if (cb < 0 || cb > 2) return fail(EXL3_EINVAL, "invalid EXL3 codebook %d", cb);
  if (!trellis || in <= 0 || in % 16 || bank_tiles <= 0)
    return fail(EXL3_EINVAL, "invalid expert trellis");
  if (out <= 0 || out % 128) return fail(EXL3_EINVAL, "expert output width must be 128-aligned");
  if (projections <= 0 || routes <= 0 || (int64_t)routes * projections != rows)
    return fail(EXL3_EINVAL, "expert route count does not match input rows");
  if (!selected || !suh) return fail(EXL3_EINVAL, "invalid expert routes or input scales");
  if (!raw && !svh) return fail(EXL3_EINVAL, "invalid expert output scales");
  // the input Hadamard needs whole 128-blocks; the bank must hold every
  // projection's columns of a route (the expert index is checked per row on
  // the device: rows past the bank produce zeros)
  if (in % 128) return fail(EXL3_EINVAL, "expert input width must be 128-aligned");
  if (stride_tiles < 0 ||
      (int64_t)(projections - 1) * stride_tiles + out / 16 > (int64_t)bank_tiles)
    return fail(EXL3_EINVAL, "expert tile map outside the bank");
  if (x_type != EXL3_F16 && x_type != EXL3_BF16 && x_type != EXL3_F32)
    return fail(EXL3_EINVAL, "unsupported expert input dtype %d", x_type);
  if (!x || !y) return fail(EXL3_EINVAL, "null expert input or output");
  if (rows > INT32_MAX / std::max(in, out) || rows * (out / 128) > INT32_MAX)
    return fail(EXL3_EINVAL, "expert input too large: %lld rows", (long long)rows);
  const size_t need = exl3_expert_mapped_workspace_bytes(in, out, rows);
  if (!workspace || workspace_bytes < need)
    return fail(EXL3_EINVAL, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace + kWorkspaceCounterBytes;
  uint16_t* xhat = (uint16_t*)ws;
  float* partials = (float*)(ws + align256((size_t)rows * in * 2));

  if (int rc = launch_gate("expert prologue")) return rc;
  PrologueParams pp{};
  pp.x = x;
  pp.x_dtype = x_type;
  pp.in = in;
  pp.rows = (int)rows;
  pp.suh[0] = suh;
  pp.xhat[0] = xhat;
  pp.suh_stride = (size_t)in;
  launch_prologue(pp, 1, s);
  if (int rc = check_launch("expert prologue")) return rc;

  MappedParams p;
  p.trellis = (const uint32_t*)trellis;
  p.xhat = xhat;
  p.selected = selected;
  p.partials = partials;
  p.in = in;
  p.out = out;
  p.bank_tiles = bank_tiles;
  p.projections = projections;
  p.stride_tiles = stride_tiles;
  p.rows = (int)rows;
  p.splits = mapped_splits(in);
  const unsigned blocks = (unsigned)(rows * (out / 128));
  hipLaunchKernelGGL(kMapped[k - 1][cb], dim3(blocks, (unsigned)p.splits), dim3(256), 0, s, p);
  if (int rc = check_launch("expert QMV")) return rc;
  hipLaunchKernelGGL(mapped_finish, dim3(blocks), dim3(64), 0, s, (const float*)partials,
                     (int)rows, out, p.splits, svh, raw, (int)x_type, y);
  return check_launch("expert finish");
}

#endif  // __HIP_DEVICE_COMPILE__
