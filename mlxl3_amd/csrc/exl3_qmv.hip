// Instantiations of the multi-row QMV and the decode hook over K x codebook.
#include "exl3_launch.hpp"
#include "exl3_qmv.hpp"

namespace exl3 {

#define EXL3_QMV_INST(K, CB)                                                \
  template __global__ void qmv_kernel<K, CB, 1, false, false>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 1, false, false, true>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 2, false, false, true>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 1, true, false>(QmvParams);  \
  template __global__ void qmv_kernel<K, CB, 1, true, true>(QmvParams);   \
  template __global__ void qmv_kernel<K, CB, 1, true, false, true>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 1, true, true, true>(QmvParams); \
  template __global__ void qmv_kernel<K, CB, 2, true, false>(QmvParams);  \
  template __global__ void qmv_kernel<K, CB, 4, true, false>(QmvParams);
#define EXL3_DEC_INST(K, CB)                                                             \
  template __global__ void decode_tiles_kernel<K, CB>(const uint32_t*, int64_t, uint16_t*, \
                                                      uint16_t*);
EXL3_INSTANTIATE(EXL3_QMV_INST)
EXL3_INSTANTIATE(EXL3_DEC_INST)
template __global__ void codewords_kernel<0>(const uint16_t*, int64_t, uint16_t*);
template __global__ void codewords_kernel<1>(const uint16_t*, int64_t, uint16_t*);
template __global__ void codewords_kernel<2>(const uint16_t*, int64_t, uint16_t*);

// Packing, the inverse of the tile decode on the low K bits of each state
// (codec::pack, codec.rs:73-100; GPU form exl3_pack, exl3.metal:85-100): the
// stored word at index i of a tile holds logical word i ^ 1 (the u32 halves
// swapped), whose 16 bits are the stream bits 16*(l % K) .. +15 of the span
// l / K of 16 states, taken most significant first.  One thread per stored
// word; the tile's 256 states (512 bytes) sit in L1 for its 16K threads.
__global__ __launch_bounds__(256) void pack_tiles_kernel(const uint16_t* __restrict__ states,
                                                         int64_t words, int k,
                                                         uint16_t* __restrict__ packed) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t tile = i / (16 * k);
  const int logical = (int)(i - tile * 16 * k) ^ 1;
  const uint16_t* span = states + tile * 256 + (logical / k) * 16;
  const int first = (logical % k) * 16;  // first stream bit of this word
  uint32_t word = 0;
  for (int bit = 0; bit < 16; ++bit) {
    const int sb = first + bit;
    word = (word << 1) | ((span[sb / k] >> (k - 1 - sb % k)) & 1u);
  }
  packed[i] = (uint16_t)word;
}

// Inner product of a decoded trellis without glue (the reference's serial
// exl3_qmv, exl3.metal:118-142): y[n] = f16(sum_r x[r] * W[r][n]), W read from
// the decoded tiles `values` ([tile][256] in stored order) through the tile
// permutation (codec.rs:126-138: stored index 8*lane + 4*cg + ri holds row
// {r0, r0+1, r0+8, r0+9}[ri], column lane/4 + 8*cg, r0 = 2*(lane%4)).  One
// wave per column: lanes take rows lane, lane+64, ... in f32 and meet in a
// fixed butterfly order.
__global__ __launch_bounds__(256) void qmv_inner_kernel(const uint16_t* __restrict__ values,
                                                        const uint16_t* __restrict__ x, int rows,
                                                        int cols, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= cols) return;  // uniform per wave
  const int tn = n >> 4, c = n & 15;
  const int cg = c >> 3, c0 = c & 7;
  float acc = 0.f;
  for (int r = lane; r < rows; r += 64) {
    const int rr = r & 15;
    const int ri = (rr & 1) | ((rr >> 3) << 1), r0 = rr & 6;
    const int t = 8 * (4 * c0 + (r0 >> 1)) + 4 * cg + ri;
    const int64_t tile = (int64_t)(r >> 4) * (cols >> 4) + tn;
    acc = fmaf(h2f(x[r]), h2f(values[tile * 256 + t]), acc);
  }
  acc += xor_lanes<1>(acc);
  acc += xor_lanes<2>(acc);
  acc += xor_lanes<4>(acc);
  acc += xor_lanes<8>(acc);
  acc += xor_lanes<16>(acc);
  acc += xor_lanes<32>(acc);
  if (lane == 0) y[n] = f2h(acc);
}


// Host-side launchers (not part of the device compilation pass).
#ifndef __HIP_DEVICE_COMPILE__
template <int K, int CB>
static void run_qmv1s(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1, false, false>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv1s_shallow(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1, false, false, true>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv2s_shallow(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 2, false, false, true>), grid, dim3(512), lds, s, p);
}
template <int K, int CB>
static void run_qmv1(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1, true, false>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv1f(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1, true, true>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv1_shallow(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1, true, false, true>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv1f_shallow(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 1, true, true, true>), grid, dim3(256), lds, s, p);
}
template <int K, int CB>
static void run_qmv2(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 2, true, false>), grid, dim3(512), lds, s, p);
}
template <int K, int CB>
static void run_qmv4(const QmvParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((qmv_kernel<K, CB, 4, true, false>), grid, dim3(1024), lds, s, p);
}
template <int K, int CB>
static void run_decode(const uint32_t* packed, int64_t tiles, uint16_t* st, uint16_t* val,
                       dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_tiles_kernel<K, CB>), grid, dim3(256), 0, s, packed, tiles, st, val);
}

void launch_codewords(const uint16_t* states, int64_t n, int cb, uint16_t* values,
                      hipStream_t s) {
  const dim3 grid((unsigned)((n + 255) / 256));
  if (cb == 0) hipLaunchKernelGGL((codewords_kernel<0>), grid, dim3(256), 0, s, states, n, values);
  else if (cb == 1) hipLaunchKernelGGL((codewords_kernel<1>), grid, dim3(256), 0, s, states, n, values);
  else hipLaunchKernelGGL((codewords_kernel<2>), grid, dim3(256), 0, s, states, n, values);
}

void launch_pack_tiles(const uint16_t* states, int64_t tiles, int k, uint16_t* packed,
                       hipStream_t s) {
  const int64_t words = tiles * 16 * k;
  hipLaunchKernelGGL(pack_tiles_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s,
                     states, words, k, packed);
}

void launch_qmv_inner(const uint16_t* values, const uint16_t* x, int rows, int cols, uint16_t* y,
                      hipStream_t s) {
  hipLaunchKernelGGL(qmv_inner_kernel, dim3((unsigned)((cols + 3) / 4)), dim3(256), 0, s, values,
                     x, rows, cols, y);
}

const QmvFn kQmv[3][8][3] = {EXL3_TABLE(run_qmv1), EXL3_TABLE(run_qmv2), EXL3_TABLE(run_qmv4)};
const QmvFn kQmvSingle[8][3] = EXL3_TABLE(run_qmv1s);
const QmvFn kQmvSingleShallow[8][3] = EXL3_TABLE(run_qmv1s_shallow);
const QmvFn kQmvSingle2[8][3] = EXL3_TABLE(run_qmv2s_shallow);
const QmvFn kQmvFrag[8][3] = EXL3_TABLE(run_qmv1f);
const QmvFn kQmvShallow[8][3] = EXL3_TABLE(run_qmv1_shallow);
const QmvFn kQmvFragShallow[8][3] = EXL3_TABLE(run_qmv1f_shallow);
const DecodeFn kDecode[8][3] = EXL3_TABLE(run_decode);

#endif

}  // namespace exl3

#ifdef EXL3_QMV_PHASES
// The phase-probe build's stamp buffer for the single-row QMV (a device
// pointer with room for kPhaseWords words per wave of a launch, or NULL to
// stop recording).  Not part of the library's ABI: only this build has it.
extern "C" int exl3_debug_phase_buffer(void* dev) {
  return hipMemcpyToSymbol(HIP_SYMBOL(exl3::qmv_phase_out), &dev, sizeof(dev)) == hipSuccess ? 0
                                                                                             : -2;
}
#endif

