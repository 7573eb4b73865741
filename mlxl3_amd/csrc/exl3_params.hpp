// Kernel parameter blocks (plain structs passed by value to the kernels).
#pragma once

#include <stdint.h>

namespace exl3 {

struct QmvParams {
  const uint32_t* trellis;  // [in/16][out/16][8K] u32
  const void* x;            // [M][in] of x_dtype
  const uint16_t* suh;      // [in] f16
  const uint16_t* svh;      // [out] f16
  const uint16_t* bias;     // [out] f16 or null
  void* y;                  // [M][out] of y_dtype
  float* partials;          // [splits][M][out]
  uint32_t* counters;       // [out/128], zero between calls
  int in, out, M, splits;
  int x_dtype, y_dtype;
};

struct QmmParams {
  const uint32_t* trellis;  // [in/16][out/16][8K] u32
  const uint16_t* xhat;     // [M][in] f16 (prologue output)
  const uint16_t* svh;      // [out]
  const uint16_t* bias;     // [out] or null
  void* y;                  // [M][out]
  float* partials;          // [splits][M][out] f32 (splits > 1)
  uint32_t* counters;       // [mtiles * col_blocks], zero between calls (splits > 1)
  int in, out, M, y_dtype;
  int col_blocks;           // out / 128
  int mtiles;               // ceil(M / rows per workgroup)
  int splits;               // K-ranges per output tile (global split-K)
};

}  // namespace exl3
