// Instantiations of the prologue and the QMM over K x codebook x row tile.
#include "exl3_launch.hpp"
#include "exl3_qmm.hpp"

namespace exl3 {

#define EXL3_QMM_INST(K, CB)                                   \
  template __global__ void qmm_kernel<K, CB, 1>(QmmParams); \
  template __global__ void qmm_kernel<K, CB, 2>(QmmParams); \
  template __global__ void qmm_kernel<K, CB, 4>(QmmParams);
EXL3_INSTANTIATE(EXL3_QMM_INST)

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

void launch_prologue(const void* x, int x_dtype, const uint16_t* suh, int in, int rows,
                     uint16_t* xhat, hipStream_t s) {
  const int64_t waves = (int64_t)rows * ((in / 128 + 7) / 8);
  hipLaunchKernelGGL(prologue_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x,
                     x_dtype, suh, in, rows, xhat);
}

void launch_fill_zero(uint32_t* p, size_t words, hipStream_t s) {
  unsigned blocks = (unsigned)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, s, p, words);
}

#endif

}  // namespace exl3
