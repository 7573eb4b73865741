// Instantiations of the multi-row QMV and the decode hook over K x codebook.
#include "exl3_launch.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {

#define EXL3_QMV_INST(K, CB)                                  \
  template __global__ void qmv_kernel<K, CB, 1>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 2>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 4>(QmvParams);
#define EXL3_DEC_INST(K, CB)                                                             \
  template __global__ void decode_tiles_kernel<K, CB>(const uint32_t*, int64_t, uint16_t*, \
                                                      uint16_t*);
EXL3_INSTANTIATE(EXL3_QMV_INST)
EXL3_INSTANTIATE(EXL3_DEC_INST)

// Host-side launchers (not part of the device compilation pass).
#ifndef __HIP_DEVICE_COMPILE__
template <int K, int CB>
static void run_qmv1(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv2(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 2>), grid, dim3(512), lds, s, p);
}
template <int K, int CB>
static void run_qmv4(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 4>), grid, dim3(1024), lds, s, p);
}
template <int K, int CB>
static void run_decode(const uint32_t* packed, int64_t tiles, uint16_t* st, uint16_t* val,
                       dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_tiles_kernel<K, CB>), grid, dim3(256), 0, s, packed, tiles, st, val);
}

const QmvFn kQmv[3][8][3] = {EXL3_TABLE(run_qmv1), EXL3_TABLE(run_qmv2), EXL3_TABLE(run_qmv4)};
const DecodeFn kDecode[8][3] = EXL3_TABLE(run_decode);

#endif

}  // namespace exl3
