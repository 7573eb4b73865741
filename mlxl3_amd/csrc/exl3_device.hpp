// Device-side building blocks for the EXL3 quantized linear on gfx950.
//
// Trellis tile layout (the reference's on-disk and in-memory format,
// native/src/codec.rs:40-50): a 16x16 tile of K-bit symbols is a circular
// 256*K-bit stream stored as 8*K little-endian u32 words; stream bit 0 is the
// MSB of word 0.  The 16-bit state of weight t is the window that ends
// (exclusive) at stream bit (t+1)*K.  Tiles sit at [in/16][out/16] in
// row-major tile order, so the 8*K words of one tile are contiguous.
//
// Lane ownership used by every kernel here: a tile is read by 8 consecutive
// lanes, lane j holding words [j*K, j*K+K) (one K-dword load).  Because the
// state windows end every K bits, lane j owns exactly the 32 states
// [32j, 32j+32), whose windows lie in its own K words plus the 16-K bits at
// the end of the previous lane's last word.  Through the tile permutation
// (codec.rs:126-138) those 32 states are all 16 rows of columns j and j+8.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace exl3 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

constexpr float kHadScale = 0.08838834764831845f;  // f32 bits 0x3db504f3

// ---------------------------------------------------------------------------
// compile-time loop helper
// ---------------------------------------------------------------------------
template <int... Is, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// acc + v where `live`, else acc, as a select.  Sums over a chunk of values
// loaded together (split-K partials, top-k slots) add them with this: behind a
// conditional add the compiler sinks each load into its branch, and the chunk's
// loads then go out one round trip at a time.
__device__ __forceinline__ float add_if(bool live, float acc, float v) {
  const float s = acc + v;
  return live ? s : acc;
}
__device__ __forceinline__ float4v add_if(bool live, float4v acc, float4v v) {
  const float4v s = acc + v;
  return live ? s : acc;
}

// ---------------------------------------------------------------------------
// f16 helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float round_f16(float v) { return (float)(_Float16)v; }
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float bf2f(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

enum : int { DT_F16 = 9, DT_F32 = 10, DT_BF16 = 12 };

// Output conversion of the linear epilogue (linear.rs:992-995): the f16 value
// is cast to the activation dtype x_dt, then the f16 bias is added with MLX's
// type promotion -- f16 + f16 in f16, f32 + f16 in f32, and bf16 + f16 in f32
// (MLX promotes the pair to float32).  y_dt is that result dtype: x_dt without
// a bias, f32 for bf16 activations with a bias (the host checks it).
__device__ __forceinline__ float out_value(int x_dt, float v16, const uint16_t* bias, int col) {
  float v = x_dt == DT_BF16 ? bf2f(f2bf(v16)) : v16;
  if (bias) v = x_dt == DT_F16 ? round_f16(v + h2f(bias[col])) : v + h2f(bias[col]);
  return v;
}
__device__ __forceinline__ void store_out(void* p, int y_dt, int x_dt, size_t i, float v16,
                                          const uint16_t* bias, int col) {
  const float v = out_value(x_dt, v16, bias, col);
  if (y_dt == DT_F16)
    ((uint16_t*)p)[i] = f2h(v);
  else if (y_dt == DT_BF16)
    ((uint16_t*)p)[i] = f2bf(v);
  else
    ((float*)p)[i] = v;
}

// ---------------------------------------------------------------------------
// state windows
// ---------------------------------------------------------------------------
// B[0] is the previous lane's last word, B[1..K] the lane's own words.  The
// window of local state s starts at bit (s+1)*K + 16 of B (big-endian).

// 16-bit window of state S in the low half of the result (upper bits junk).
template <int K, int S>
__device__ __forceinline__ uint32_t window16(const uint32_t* B) {
  constexpr int beta = (S + 1) * K + 16;
  constexpr int a = beta >> 5, o = beta & 31;
  if constexpr (o <= 16)
    return B[a] >> (16 - o);
  else
    return __builtin_amdgcn_alignbit(B[a], B[a + 1], 48 - o);
}

// 32-bit window starting at state S: hi16 = state S, lo16 = state S + 16/K.
template <int K, int S>
__device__ __forceinline__ uint32_t window32(const uint32_t* B) {
  constexpr int beta = (S + 1) * K + 16;
  constexpr int a = beta >> 5, o = beta & 31;
  if constexpr (o == 0)
    return B[a];
  else
    return __builtin_amdgcn_alignbit(B[a], B[a + 1], 32 - o);
}

// For K in {1,2,4,8} states S and S+16/K share one 32-bit window.
template <int K, int S>
constexpr int state_half() {
  if constexpr (16 % K == 0) {
    constexpr int d = 16 / K;
    return ((S / d) % 2 == 0) ? 1 : 0;
  } else {
    return 0;
  }
}

template <int K>
__device__ __forceinline__ void extract_states(const uint32_t* B, uint32_t (&src)[32]) {
  static_for<32>([&](auto S_) {
    constexpr int S = decltype(S_)::value;
    if constexpr (16 % K == 0) {
      constexpr int d = 16 / K;
      if constexpr ((S / d) % 2 == 0)
        src[S] = window32<K, S>(B);
      else
        src[S] = src[S - d];
    } else {
      src[S] = window16<K, S>(B);
    }
  });
}

template <int K, int S>
__device__ __forceinline__ uint32_t state_value(const uint32_t (&src)[32]) {
  return state_half<K, S>() ? (src[S] >> 16) : (src[S] & 0xffffu);
}

// ---------------------------------------------------------------------------
// procedural codebooks (codec.rs:52-71)
// ---------------------------------------------------------------------------
// Step 1, the 32-bit multiply of the 16-bit state (taken from the low or high
// half of w), done with full-rate 16/24-bit multiplies:
//   3INST: x*89226354 + 64248484 = (x*6)*14871059 + 64248484   (x*6 < 2^24)
//   MCG/MUL1: x*a = x*a_lo + ((x*a_hi mod 2^16) << 16)          (mod 2^32)
template <int HI>
__device__ __forceinline__ uint32_t mad_u32_u16(uint32_t w, uint32_t b, uint32_t c) {
  uint32_t d;
  if constexpr (HI)
    asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(d) : "v"(w), "v"(b), "v"(c));
  else
    asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(d) : "v"(w), "v"(b), "v"(c));
  return d;
}

template <int HI>
__device__ __forceinline__ uint32_t mul_u24_to_hi16(uint32_t w, uint32_t b) {
  uint32_t d;
  if constexpr (HI)
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 "
        "src1_sel:DWORD"
        : "=v"(d)
        : "v"(w), "v"(b));
  else
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 "
        "src1_sel:DWORD"
        : "=v"(d)
        : "v"(w), "v"(b));
  return d;
}

__device__ __forceinline__ uint32_t mad_u32_u24(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(b), "v"(c));
  return d;
}

template <int CB, int HI>
__device__ __forceinline__ uint32_t codeword_product(uint32_t w) {
  if constexpr (CB == 0) {
    uint32_t t = mad_u32_u16<HI>(w, 6u, 0u);
    return mad_u32_u24(t, 14871059u, 64248484u);
  } else if constexpr (CB == 1) {
    uint32_t t = mul_u24_to_hi16<HI>(w, 0xcbacu);
    return mad_u32_u16<HI>(w, 0x1fedu, t);
  } else {
    uint32_t t = mul_u24_to_hi16<HI>(w, 0x83dcu);
    return mad_u32_u16<HI>(w, 0xd12du, t);
  }
}

// binary16 sum of the two halves of z written to the low half (high zeroed) or
// to the high half (low half of `into` kept).
__device__ __forceinline__ uint32_t add_halves_lo(uint32_t z) {
  uint32_t d;
  asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 "
      "src1_sel:WORD_1"
      : "=v"(d)
      : "v"(z));
  return d;
}
__device__ __forceinline__ uint32_t add_halves_hi(uint32_t z, uint32_t into) {
  uint32_t d = into;
  asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 "
      "src1_sel:WORD_1"
      : "+v"(d)
      : "v"(z));
  return d;
}

__device__ __forceinline__ uint32_t byte_sum_plus_6400(uint32_t y) {
  uint32_t d;
  asm("v_sad_u8 %0, %1, 0, %2" : "=v"(d) : "v"(y), "v"(0x6400u));
  return d;
}

// Two decoded weights (states S0 and S0+1 of the lane) packed as f16x2
// (S0 in the low half).
template <int CB, int K, int S0>
__device__ __forceinline__ uint32_t decode_pair(const uint32_t (&src)[32]) {
  uint32_t y0 = codeword_product<CB, state_half<K, S0>()>(src[S0]);
  uint32_t y1 = codeword_product<CB, state_half<K, S0 + 1>()>(src[S0 + 1]);
  if constexpr (CB < 2) {
    uint32_t z0 = (y0 & 0x8fff8fffu) ^ 0x3b603b60u;
    uint32_t z1 = (y1 & 0x8fff8fffu) ^ 0x3b603b60u;
    return add_halves_hi(z1, add_halves_lo(z0));
  } else {
    // f16(h * 0x1eee + 0xc931) with one rounding (codec.rs:57-65): fused
    // multiply-add on the packed pair of sums.
    uint32_t s0 = byte_sum_plus_6400(y0), s1 = byte_sum_plus_6400(y1);
    half2v h = __builtin_bit_cast(half2v, s0 | (s1 << 16));
    const half2v inv = __builtin_bit_cast(half2v, 0x1eee1eeeu);
    const half2v bias = __builtin_bit_cast(half2v, 0xc931c931u);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(h, inv, bias));
  }
}

// Single weight, f16 bits in the low half.
template <int CB, int K, int S>
__device__ __forceinline__ uint32_t decode_one(const uint32_t (&src)[32]) {
  uint32_t y = codeword_product<CB, state_half<K, S>()>(src[S]);
  if constexpr (CB < 2) {
    return add_halves_lo((y & 0x8fff8fffu) ^ 0x3b603b60u);
  } else {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)byte_sum_plus_6400(y));
    _Float16 r = __builtin_elementwise_fma(h, __builtin_bit_cast(_Float16, (uint16_t)0x1eee),
                                           __builtin_bit_cast(_Float16, (uint16_t)0xc931));
    return __builtin_bit_cast(uint16_t, r);
  }
}

// Gather the previous lane's last word within each group of 8 lanes.
__device__ __forceinline__ uint32_t prev_word(uint32_t last, int lane) {
  int src = (lane & ~7) | ((lane + 7) & 7);
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)last);
}

// ---------------------------------------------------------------------------
// MFMA B fragments for one tile pair
// ---------------------------------------------------------------------------
// For v_mfma_f32_16x16x32_f16 a lane l holds B[k][n] for n = l%16 and the
// eight k slots of lane group l/16.  A lane decodes rows 0..15 of columns j
// and j+8; fragment (h, cg) takes rows 8h..8h+7 of column j+8cg.  Row 8h+2p
// and 8h+2p+1 of column j+8cg are local states 8p+4cg+2h and +1, so dword p
// of the fragment is decode_pair at S0 = 8p + 4cg + 2h.
template <int CB, int K, int H, int CG>
__device__ __forceinline__ half8 decode_fragment(const uint32_t (&src)[32]) {
  u32x4 d;
  d[0] = decode_pair<CB, K, 0 + 4 * CG + 2 * H>(src);
  d[1] = decode_pair<CB, K, 8 + 4 * CG + 2 * H>(src);
  d[2] = decode_pair<CB, K, 16 + 4 * CG + 2 * H>(src);
  d[3] = decode_pair<CB, K, 24 + 4 * CG + 2 * H>(src);
  return __builtin_bit_cast(half8, d);
}

// Two B fragments written by the decode's inline assembly, passed through one
// `s_nop 1` on their way to the MFMAs.  A VALU write of a VGPR needs 2 wait
// states before an MFMA reads that VGPR; the compiler inserts them only for
// writes it can see, and the decode's SDWA adds are inline assembly to it.
// Without this some schedules left 1 wait state between the last half-write of
// a fragment and its MFMA, which then read the register's previous value
// (wrong, run-to-run varying partial sums of the second tile of a pair).
// The statement is volatile: as a plain asm statement the scheduler was free to
// move it, and the schedules it chose were slower (NS QMV 14.06 -> 15.85 us).
__device__ __forceinline__ void mfma_operand_fence(half8& b0, half8& b1) {
  asm volatile("s_nop 1" : "+v"(b0), "+v"(b1));
}

__device__ __forceinline__ float4v mfma16(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// lane exchanges: value of lane (lane ^ S) within the wave
// ---------------------------------------------------------------------------
// S = 1, 2: DPP quad permutations; 4: the half-row mirror composed with a
// quad reversal (i^7^3 = i^4); 8: a rotation by 8 inside the 16-lane row; 16:
// a ds_swizzle in bit-mask mode (xor 0x10 inside 32 lanes); 32: ds_bpermute.
template <int S>
__device__ __forceinline__ float xor_lanes(float v) {
  const int b = __builtin_bit_cast(int, v);
  int r;
  if constexpr (S == 1) {
    r = __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (S == 2) {
    r = __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (S == 4) {
    int t = __builtin_amdgcn_update_dpp(0, b, 0x141, 0xF, 0xF, false);  // row_half_mirror
    r = __builtin_amdgcn_update_dpp(0, t, 0x1B, 0xF, 0xF, false);       // quad_perm [3,2,1,0]
  } else if constexpr (S == 8) {
    r = __builtin_amdgcn_update_dpp(0, b, 0x128, 0xF, 0xF, false);  // row_ror:8 = xor 8 in 16
  } else if constexpr (S == 16) {
    r = __builtin_amdgcn_ds_swizzle(b, 0x401F);  // and 0x1f, or 0, xor 0x10
  } else {
    static_assert(S == 32, "lane exchange distance");
    r = __builtin_amdgcn_ds_bpermute((int)((__lane_id() ^ 32) << 2), b);
  }
  return __builtin_bit_cast(float, r);
}

// ---------------------------------------------------------------------------
// wave-level Hadamard-128: lane holds elements lane and lane+64
// ---------------------------------------------------------------------------
// Ascending radix-2 stages (the MLX butterfly order pinned by the reference's
// hadamard fixture); STAGED rounds to f16 after the stride-8 and stride-64
// stages (exl3.metal:156-170).  The 1/sqrt(128) scale is left to the caller.
template <bool STAGED>
__device__ __forceinline__ void h128_wave(float& v0, float& v1, int lane) {
  static_for<6>([&](auto i_) {
    constexpr int stride = 1 << decltype(i_)::value;
    const float p0 = xor_lanes<stride>(v0);
    const float p1 = xor_lanes<stride>(v1);
    if (lane & stride) {
      v0 = p0 - v0;
      v1 = p1 - v1;
    } else {
      v0 = v0 + p0;
      v1 = v1 + p1;
    }
    if (STAGED && stride == 8) {
      v0 = round_f16(v0);
      v1 = round_f16(v1);
    }
  });
  float a = v0, b = v1;
  v0 = a + b;
  v1 = a - b;
  if (STAGED) {
    v0 = round_f16(v0);
    v1 = round_f16(v1);
  }
}

// Slot of a 16-byte A chunk in its LDS row: chunk c of row r sits at
// c ^ a_swizzle(r).  A fragment read (ds_read_b128, 16 rows x one chunk,
// rows 128 bytes apart) is served 16 lanes (256 bytes, all 64 banks) at a
// time on gfx950, so rows r and r + 8 (same bank offset r * 128 mod 256)
// need different slots; r & 7 alone maps them to the same one (a 2-way
// conflict that halved the read rate, 128 vs 256 B/clk measured).
__device__ __forceinline__ int a_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector memory
// instructions of the wave are outstanding and leaves the other counters free.
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Buffer resource word 3 for raw dword buffer accesses on gfx9-family GPUs,
// and the cache-policy operand of a coherent (sc1: agent scope, served by the
// coherence point) buffer access.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kCpolSc1 = 16;
// Cache-policy operand of a streaming (non-temporal) buffer load.
constexpr int kCpolNt = 2;

// Byte offset of an LDS location in the workgroup's allocation.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// global_load_lds_dwordx4 as inline assembly, in its scalar-base form: lane
// l copies the 16 bytes at base + off (base wave-uniform, off the lane's
// 32-bit byte offset) into LDS bytes lds + 16l .. lds + 16l + 15 (lds
// wave-uniform; the s_nop covers the M0 write -> LDS-DMA hazard).  The
// compiler does not see this LDS write, so it adds no waits of its own for it
// (it cannot tell the destination from other LDS accesses and would wait for
// every outstanding load before them): the caller waits with s_waitcnt vmcnt
// before the barrier that publishes the bytes.  "memory" keeps other memory
// accesses from moving across the issue.
__device__ __forceinline__ void lds_dma16_s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}

}  // namespace exl3
