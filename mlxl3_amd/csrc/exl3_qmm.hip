// Instantiations of the prologue and the QMM over K x codebook x row tile.
#include <algorithm>

#include "exl3_launch.hpp"
#include "exl3_qmm.hpp"

namespace exl3 {

#define EXL3_QMM_INST(K, CB)                                   \
  template __global__ void qmm_kernel<K, CB, 1>(QmmParams); \
  template __global__ void qmm_kernel<K, CB, 2>(QmmParams); \
  template __global__ void qmm_kernel<K, CB, 4>(QmmParams);
EXL3_INSTANTIATE(EXL3_QMM_INST)
template __global__ void prologue_kernel<true>(PrologueParams);
template __global__ void prologue_kernel<false>(PrologueParams);
template __global__ void swiglu_prepare_kernel<true>(const uint16_t*, const uint16_t*,
                                                     const uint16_t*, int, int, uint16_t*);
template __global__ void swiglu_prepare_kernel<false>(const uint16_t*, const uint16_t*,
                                                      const uint16_t*, int, int, uint16_t*);

// out = swiglu(gate, up) or geglu(gate, up) elementwise in f16, eight
// elements per thread where the buffers allow 16-byte access.
template <bool GELU>
__device__ __forceinline__ float glu_f16(float g, float u) {
  if constexpr (GELU) return geglu_f16(g, u);
  else return swiglu_f16(g, u);
}
template <bool GELU>
__global__ __launch_bounds__(256) void glu_kernel(const uint16_t* __restrict__ g,
                                                  const uint16_t* __restrict__ u,
                                                  uint16_t* __restrict__ o, int64_t n, int vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    for (; i < n / 8; i += stride) {
      const u32x4 gv = ((const u32x4*)g)[i], uv = ((const u32x4*)u)[i];
      u32x4 ov;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = glu_f16<GELU>(h2f((uint16_t)gv[j]), h2f((uint16_t)uv[j]));
        const float hi = glu_f16<GELU>(h2f((uint16_t)(gv[j] >> 16)), h2f((uint16_t)(uv[j] >> 16)));
        ov[j] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
      }
      ((u32x4*)o)[i] = ov;
    }
    i = n / 8 * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  }
  for (; i < n; i += stride) o[i] = f2h(glu_f16<GELU>(h2f(g[i]), h2f(u[i])));
}
template __global__ void glu_kernel<false>(const uint16_t*, const uint16_t*, uint16_t*, int64_t,
                                           int);
template __global__ void glu_kernel<true>(const uint16_t*, const uint16_t*, uint16_t*, int64_t,
                                          int);

__global__ void fill_zero_kernel(uint32_t* p, size_t words) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < words; i += stride) p[i] = 0u;
}

// Host-side launchers (not part of the device compilation pass).
#ifndef __HIP_DEVICE_COMPILE__
template <int K, int CB, int MB>
static void run_qmm(const QmmParams& p, dim3 g, hipStream_t s) {
  hipLaunchKernelGGL((qmm_kernel<K, CB, MB>), g, dim3(512), 0, s, p);
}
template <int K, int CB>
static void run_qmm1(const QmmParams& p, dim3 g, hipStream_t s) {
  run_qmm<K, CB, 1>(p, g, s);
}
template <int K, int CB>
static void run_qmm2(const QmmParams& p, dim3 g, hipStream_t s) {
  run_qmm<K, CB, 2>(p, g, s);
}
template <int K, int CB>
static void run_qmm4(const QmmParams& p, dim3 g, hipStream_t s) {
  run_qmm<K, CB, 4>(p, g, s);
}

const QmmFn kQmm[3][8][3] = {EXL3_TABLE(run_qmm1), EXL3_TABLE(run_qmm2), EXL3_TABLE(run_qmm4)};

void launch_prologue(const PrologueParams& p, int members, hipStream_t s) {
  const int64_t groups = ((int64_t)p.rows * (p.in / 128) + 15) / 16;
  // prologue_kernel indexes jobs in 32 bits: the entry points reject
  // rows * in > INT32_MAX, so rows * blocks stays below 2^24
  uintptr_t bits = (uintptr_t)p.x;
  for (int i = 0; i < members; ++i) bits |= (uintptr_t)p.suh[i] | (uintptr_t)p.xhat[i];
  if ((bits & 15) == 0)
    hipLaunchKernelGGL(prologue_kernel<true>, dim3((unsigned)groups, (unsigned)members),
                       dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(prologue_kernel<false>, dim3((unsigned)groups, (unsigned)members),
                       dim3(256), 0, s, p);
}

void launch_glu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, bool gelu,
                hipStream_t s) {
  const int vec = ((((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) & 15) == 0) ? 1 : 0;
  const int64_t work = vec ? n / 8 + 8 : n;
  const unsigned blocks = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
  if (gelu)
    hipLaunchKernelGGL(glu_kernel<true>, dim3(blocks), dim3(256), 0, s, gate, up, out, n, vec);
  else
    hipLaunchKernelGGL(glu_kernel<false>, dim3(blocks), dim3(256), 0, s, gate, up, out, n, vec);
}

void launch_swiglu_prepare(const uint16_t* gate, const uint16_t* up, const uint16_t* down_suh,
                           int H, int rows, uint16_t* xhat, hipStream_t s) {
  const unsigned groups = (unsigned)(((int64_t)rows * (H / 128) + 15) / 16);
  if ((((uintptr_t)gate | (uintptr_t)up | (uintptr_t)down_suh | (uintptr_t)xhat) & 15) == 0)
    hipLaunchKernelGGL(swiglu_prepare_kernel<true>, dim3(groups), dim3(256), 0, s, gate, up,
                       down_suh, H, rows, xhat);
  else
    hipLaunchKernelGGL(swiglu_prepare_kernel<false>, dim3(groups), dim3(256), 0, s, gate, up,
                       down_suh, H, rows, xhat);
}

void launch_fill_zero(uint32_t* p, size_t words, hipStream_t s) {
  unsigned blocks = (unsigned)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, s, p, words);
}

#endif

}  // namespace exl3
