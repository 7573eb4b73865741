/*
 * CPU oracle for the EXL3 quantized-linear path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker or the timed CPU baseline.  The
 * shipped library (mlxl3_amd/libexl3_hip.so) contains no call into it.
 *
 * Each function restates a reference algorithm; the citation is given at the
 * function.  Paths are relative to the reference tree.
 */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

float exl3o_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float v = (float)m * 0x1p-24f; /* exact: m < 2^10 */
        return sign ? -v : v;
    }
    if (e == 31)
        bits = sign | 0x7f800000u | (m << 13);
    else
        bits = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Correctly rounded (nearest, ties to even) binary64 -> binary16. */
uint16_t exl3o_f64_to_f16(double d) {
    uint16_t sign = signbit(d) ? 0x8000u : 0u;
    double a = fabs(d);
    if (a != a) return (uint16_t)(sign | 0x7e00u);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x1p-14) {
        /* subnormal quantum 2^-24; a*2^24 is exact in binary64 */
        double r = nearbyint(a * 0x1p24);
        return (uint16_t)(sign | (uint16_t)r); /* r == 1024 is the min normal */
    }
    int e;
    frexp(a, &e); /* a in [2^(e-1), 2^e) */
    int E = e - 1;
    double r = nearbyint(ldexp(a, 11 - e)); /* [1024, 2048] */
    if (r >= 2048.0) {
        r = 1024.0;
        E += 1;
    }
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)(((E + 15) << 10) | ((int)r - 1024)));
}

uint16_t exl3o_f32_to_f16(float f) { return exl3o_f64_to_f16((double)f); }

float exl3o_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t exl3o_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

static inline float h2f(uint16_t h) { return exl3o_f16_to_f32(h); }
static inline uint16_t f2h(float f) { return exl3o_f32_to_f16(f); }
static inline float rh(float f) { return h2f(f2h(f)); } /* round through f16 */

/* ------------------------------------------------------------------------ */
/* codec                                                                     */
/* ------------------------------------------------------------------------ */

/* decode_codeword, native/src/codec.rs:52-71 (same closed form as
 * ponyexl3/ref/codebook.py:195-220).  3INST and MCG: an LCG / MCG step, mask
 * 0x8fff8fff, xor 0x3b603b60, then the binary16 sum of the two halves.  MUL1:
 * sum of the four product bytes + 0x6400 read as binary16, then one fused
 * multiply-add with 0x1eee and 0xc931 rounded once. */
uint16_t exl3o_codeword(uint16_t state, int cb) {
    uint32_t x = state;
    if (cb == 2) {
        uint32_t p = x * 0x83dcd12du;
        uint32_t s = 0x6400u + (p & 255u) + ((p >> 8) & 255u) + ((p >> 16) & 255u) + (p >> 24);
        double h = (double)h2f((uint16_t)s);
        double inv = (double)h2f(0x1eeeu);
        double bias = (double)h2f(0xc931u);
        return exl3o_f64_to_f16(h * inv + bias); /* product and sum exact in binary64 */
    }
    uint32_t y = (cb == 0) ? x * 89226354u + 64248484u : x * 0xcbac1fedu;
    y = 0x3b603b60u ^ (y & 0x8fff8fffu);
    double lo = (double)h2f((uint16_t)(y & 0xffffu));
    double hi = (double)h2f((uint16_t)(y >> 16));
    return exl3o_f64_to_f16(lo + hi);
}

void exl3o_codebook(int cb, uint16_t* out) {
    for (uint32_t s = 0; s < 65536u; ++s) out[s] = exl3o_codeword((uint16_t)s, cb);
}

/* Tile bitstream: 32-bit word i is the little-endian pair (u16[2i], u16[2i+1])
 * (packed_pair, codec.rs:48-50); stream bit 0 is the MSB of word 0.  The state
 * of weight t is the 16-bit window ending (exclusive) at bit (t+1)*k of the
 * circular 256k-bit stream (unpack_window, codec.rs:40-46). */
static inline uint32_t tile_word(const uint16_t* tile, int k, int64_t i) {
    int64_t w = i % (8 * k);
    if (w < 0) w += 8 * k;
    return (uint32_t)tile[2 * w] | ((uint32_t)tile[2 * w + 1] << 16);
}

static void unpack_tile(const uint16_t* tile, int k, uint16_t* states) {
    const int64_t total = 256 * (int64_t)k;
    for (int t = 0; t < 256; ++t) {
        int64_t b0 = ((int64_t)(t + 1) * k - 16 + total) % total; /* first bit of window */
        int64_t i0 = b0 / 32;
        int64_t b1 = b0 + 16; /* exclusive end, unwrapped */
        int64_t i1 = (b1 - 1) / 32;
        uint64_t pair = ((uint64_t)tile_word(tile, k, i0) << 32) | tile_word(tile, k, i1);
        int shift = (int)((i1 + 1) * 32 - b1); /* i0 == i1 gives (w<<32|w) >> shift */
        states[t] = (uint16_t)(pair >> shift);
    }
}

int exl3o_unpack(const uint16_t* packed, int64_t tiles, int k, uint16_t* states) {
    if (k < 1 || k > 8 || tiles < 0) return -1;
    for (int64_t t = 0; t < tiles; ++t) unpack_tile(packed + t * 16 * k, k, states + t * 256);
    return 0;
}

/* pack, codec.rs:73-100 with pack_source :34-38: output u16 word `logical`
 * (stored at logical^1, i.e. the u32 halves swapped) collects 16 stream bits
 * MSB-first; stream bit `sb` of span `logical/k` is bit (k-1-sb%k) of symbol
 * span*16 + sb/k. */
int exl3o_pack(const uint16_t* states, int64_t tiles, int k, uint16_t* packed) {
    if (k < 1 || k > 8 || tiles < 0) return -1;
    for (int64_t t = 0; t < tiles; ++t) {
        const uint16_t* in = states + t * 256;
        uint16_t* out = packed + t * 16 * k;
        for (int logical = 0; logical < 16 * k; ++logical) {
            uint32_t word = 0;
            int span = logical / k;
            for (int bit = 0; bit < 16; ++bit) {
                int sb = (logical % k) * 16 + bit;
                int index = span * 16 + sb / k;
                int shift = k - 1 - sb % k;
                word = (word << 1) | ((in[index] >> shift) & 1u);
            }
            out[logical ^ 1] = (uint16_t)word;
        }
    }
    return 0;
}

/* permutation, codec.rs:126-138 (= ponyexl3/ref/perm.py:8-26): state index
 * 8*lane + 4*cg + ri holds row {r, r+1, r+8, r+9}[ri], col {c, c+8}[cg] with
 * r = 2*(lane%4), c = lane/4. */
void exl3o_permutation(uint16_t out[256]) {
    for (int lane = 0; lane < 32; ++lane) {
        int r = (lane % 4) * 2, c = lane / 4;
        int rows[4] = {r, r + 1, r + 8, r + 9};
        for (int cg = 0; cg < 2; ++cg)
            for (int ri = 0; ri < 4; ++ri)
                out[lane * 8 + cg * 4 + ri] = (uint16_t)(rows[ri] * 16 + c + 8 * cg);
    }
}

/* reconstruct_inner, codec.rs:158-190: tile (tk, tn) = flat tile tk*(cols/16)+tn. */
int exl3o_reconstruct_inner(const uint16_t* packed, int k, int cb, int64_t rows, int64_t cols,
                            uint16_t* out) {
    if (k < 1 || k > 8 || cb < 0 || cb > 2) return -1;
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 16) return -1;
    uint16_t perm[256];
    exl3o_permutation(perm);
    int64_t tn_count = cols / 16, tiles = rows / 16 * tn_count;
    for (int64_t tile = 0; tile < tiles; ++tile) {
        uint16_t st[256];
        unpack_tile(packed + tile * 16 * k, k, st);
        int64_t r0 = tile / tn_count * 16, c0 = tile % tn_count * 16;
        for (int i = 0; i < 256; ++i) {
            int p = perm[i];
            out[(r0 + p / 16) * cols + c0 + p % 16] = exl3o_codeword(st[i], cb);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Hadamard-128                                                              */
/* ------------------------------------------------------------------------ */

static const uint32_t kScaleBits = 0x3db504f3u; /* f32(1/sqrt(128)) */
static float had_scale(void) {
    float f;
    memcpy(&f, &kScaleBits, 4);
    return f;
}

/* One radix-2 stage of the Sylvester transform: pairs (i, i+stride) with
 * (i & stride) == 0 become (a+b, a-b). */
static void butterfly_stage(float* v, int stride) {
    for (int i = 0; i < 128; ++i) {
        if (i & stride) continue;
        float a = v[i], b = v[i + stride];
        v[i] = a + b;
        v[i + stride] = a - b;
    }
}

void exl3o_h128_f32(float* v, int64_t count) {
    const float s = had_scale();
    for (int64_t base = 0; base + 128 <= count; base += 128) {
        float* b = v + base;
        for (int stride = 1; stride < 128; stride <<= 1) butterfly_stage(b, stride);
        for (int i = 0; i < 128; ++i) b[i] = b[i] * s;
    }
}

/* exl3.metal:156-170 hadamard128_canonical (rounding after strides 8 and 64),
 * equal to MLX's f16 radix-16-then-radix-8 schedule restated at
 * linear.rs:1380-1427; the caller-side scale is f16(v * f32 scale)
 * (exl3.metal:213-215). */
void exl3o_h128_staged(float* v, int64_t count) {
    const float s = had_scale();
    for (int64_t base = 0; base + 128 <= count; base += 128) {
        float* b = v + base;
        for (int stride = 1; stride < 128; stride <<= 1) {
            butterfly_stage(b, stride);
            if (stride == 8 || stride == 64)
                for (int i = 0; i < 128; ++i) b[i] = rh(b[i]);
        }
        for (int i = 0; i < 128; ++i) b[i] = rh(b[i] * s);
    }
}

/* ------------------------------------------------------------------------ */
/* forward                                                                   */
/* ------------------------------------------------------------------------ */

enum { DT_F16 = 9, DT_F32 = 10, DT_BF16 = 12 };

static float load_x(const void* x, int dt, int64_t i) {
    if (dt == DT_F16) return h2f(((const uint16_t*)x)[i]);
    if (dt == DT_BF16) return exl3o_bf16_to_f32(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

static void store_y(void* y, int dt, int64_t i, float v) {
    if (dt == DT_F16)
        ((uint16_t*)y)[i] = f2h(v);
    else if (dt == DT_BF16)
        ((uint16_t*)y)[i] = exl3o_f32_to_bf16(v);
    else
        ((float*)y)[i] = v;
}

static int valid_dtype(int dt) { return dt == DT_F16 || dt == DT_F32 || dt == DT_BF16; }

int exl3o_result_dtype(int x_dtype, int has_bias) {
    return has_bias && x_dtype == DT_BF16 ? DT_F32 : x_dtype;
}

/* finish_and_reduce's weighted value (moe.rs:604-607): f16 * f16 rounds to
 * f16; f16 * f32 and f16 * bf16 are f32 products (MLX promotes to f32). */
static float load_score(const void* scores, int dt, int64_t i) {
    if (dt == DT_F32) return ((const float*)scores)[i];
    if (dt == DT_BF16) return exl3o_bf16_to_f32(((const uint16_t*)scores)[i]);
    return h2f(((const uint16_t*)scores)[i]);
}
static float weighted(float v16, float score, int scores_dtype) {
    return scores_dtype == DT_F16 ? rh(v16 * score) : v16 * score;
}
static void store_reduced(void* y, int scores_dtype, int64_t i, float v) {
    if (scores_dtype == DT_F16)
        ((uint16_t*)y)[i] = f2h(v);
    else
        ((float*)y)[i] = v;
}

/* Engine prologue, linear.rs:847-865: x.astype(F16) * suh (f16 multiply),
 * Hadamard-128 with scale 1/sqrt(128) in MLX's f16 schedule. */
int exl3o_prologue(const void* x, int x_dtype, int64_t rows, int in, const uint16_t* suh,
                   uint16_t* xhat) {
    if (!valid_dtype(x_dtype) || in <= 0 || in % 128 || rows < 0) return -1;
    float* buf = (float*)malloc(sizeof(float) * (size_t)in);
    if (!buf) return -3;
    for (int64_t m = 0; m < rows; ++m) {
        for (int i = 0; i < in; ++i) {
            float xv = rh(load_x(x, x_dtype, m * in + i));
            buf[i] = rh(xv * h2f(suh[i])); /* exact product, one f16 rounding */
        }
        exl3o_h128_staged(buf, in);
        for (int i = 0; i < in; ++i) xhat[m * in + i] = f2h(buf[i]);
    }
    free(buf);
    return 0;
}

static uint16_t* g_tables[3];

static const uint16_t* codebook_table(int cb) {
    uint16_t* t;
#pragma omp critical(exl3o_table)
    {
        if (!g_tables[cb]) {
            uint16_t* fresh = (uint16_t*)malloc(65536 * sizeof(uint16_t));
            if (fresh) exl3o_codebook(cb, fresh);
            g_tables[cb] = fresh;
        }
        t = g_tables[cb];
    }
    return t;
}

/* Inner product yhat[m][n] = sum_k xin[m][k] * W[k][n] with W decoded tile by
 * tile at use (no dense matrix), f32 accumulation in ascending k.  xin holds
 * f32 values (already rounded where the semantics require). */
static int gemv_tiles(const float* xin, int64_t rows, const uint16_t* trellis, int in, int out,
                      int k, int cb, float* yhat, int threads) {
    const uint16_t* table = codebook_table(cb);
    if (!table) return -3;
    uint16_t perm[256];
    exl3o_permutation(perm);
    const int tk_count = in / 16, tn_count = out / 16;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#else
    (void)threads;
#endif
    int err = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int tn = 0; tn < tn_count; ++tn) {
        float* acc = (float*)calloc((size_t)rows * 16, sizeof(float));
        if (!acc) {
#pragma omp atomic write
            err = -3;
            continue;
        }
        float w[256];
        uint16_t st[256];
        for (int tk = 0; tk < tk_count; ++tk) {
            unpack_tile(trellis + ((int64_t)tk * tn_count + tn) * 16 * k, k, st);
            for (int i = 0; i < 256; ++i) w[perm[i]] = h2f(table[st[i]]);
            for (int64_t m = 0; m < rows; ++m) {
                const float* xr = xin + m * in + tk * 16;
                float* a = acc + m * 16;
                for (int r = 0; r < 16; ++r) {
                    float xv = xr[r];
                    for (int c = 0; c < 16; ++c) a[c] += xv * w[r * 16 + c];
                }
            }
        }
        for (int64_t m = 0; m < rows; ++m)
            for (int c = 0; c < 16; ++c) yhat[m * out + tn * 16 + c] = acc[m * 16 + c];
        free(acc);
    }
    return err;
}

int exl3o_forward(int mode, const void* x, int x_dtype, int64_t rows, const uint16_t* trellis,
                  int in, int out, int k, int cb, const uint16_t* suh, const uint16_t* svh,
                  const uint16_t* bias, void* y, float* yhat_out, int threads) {
    if (mode < 0 || mode > 1 || !valid_dtype(x_dtype)) return -1;
    if (k < 1 || k > 8 || cb < 0 || cb > 2 || rows < 1) return -1;
    if (in <= 0 || out <= 0 || in % 128 || out % 128) return -1;
    if (!x || !trellis || !suh || !svh || !y) return -1;
    const float s = had_scale();
    float* xin = (float*)malloc(sizeof(float) * (size_t)(rows * in));
    float* yh = (float*)malloc(sizeof(float) * (size_t)(rows * out));
    int rc = 0;
    if (!xin || !yh) {
        rc = -3;
        goto done;
    }
    if (mode == 1) {
        uint16_t* xhat = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(rows * in));
        if (!xhat) {
            rc = -3;
            goto done;
        }
        exl3o_prologue(x, x_dtype, rows, in, suh, xhat);
        for (int64_t i = 0; i < rows * in; ++i) xin[i] = h2f(xhat[i]);
        free(xhat);
    } else {
        /* forward.py:34: xh = f16(had_r_128(f32(x16) * suh)) with the scale
         * folded into the f32 Hadamard matrix; sums taken in binary64. */
        for (int64_t m = 0; m < rows; ++m)
            for (int b = 0; b < in; b += 128) {
                double v[128];
                for (int i = 0; i < 128; ++i)
                    v[i] = (double)(rh(load_x(x, x_dtype, m * in + b + i)) * h2f(suh[b + i]));
                for (int i = 0; i < 128; ++i) {
                    double acc = 0.0;
                    for (int j = 0; j < 128; ++j)
                        acc += (__builtin_popcount((unsigned)(i & j)) & 1) ? -v[j] : v[j];
                    xin[m * in + b + i] = rh((float)(acc * (double)s));
                }
            }
    }
    rc = gemv_tiles(xin, rows, trellis, in, out, k, cb, yh, threads);
    if (rc) goto done;
    if (yhat_out) memcpy(yhat_out, yh, sizeof(float) * (size_t)(rows * out));
    for (int64_t m = 0; m < rows; ++m) {
        float* row = yh + m * out;
        if (mode == 1) {
            /* linear.rs:984-997: f16(yhat) -> f16 H128 -> * svh (f16) -> astype. */
            for (int n = 0; n < out; ++n) row[n] = rh(row[n]);
            exl3o_h128_staged(row, out);
            for (int n = 0; n < out; ++n) row[n] = rh(row[n] * h2f(svh[n]));
        } else {
            /* forward.py:41-42: y = f16(xh @ w); out = f16(had_r_128(y) * svh). */
            for (int b = 0; b < out; b += 128) {
                double v[128];
                for (int i = 0; i < 128; ++i) v[i] = (double)rh(row[b + i]);
                for (int i = 0; i < 128; ++i) {
                    double acc = 0.0;
                    for (int j = 0; j < 128; ++j)
                        acc += (__builtin_popcount((unsigned)(i & j)) & 1) ? -v[j] : v[j];
                    row[b + i] = rh((float)(acc * (double)s * (double)h2f(svh[b + i])));
                }
            }
        }
        /* linear.rs:992-995: y.astype(x.dtype), then + bias (f16) under
         * MLX's promotion: f16 + f16 in f16; f32 + f16 and bf16 + f16 in f32
         * (the result of bf16 activations with a bias is f32). */
        const int y_dtype = exl3o_result_dtype(x_dtype, bias != NULL);
        for (int n = 0; n < out; ++n) {
            float v = row[n];
            if (x_dtype == DT_BF16) v = exl3o_bf16_to_f32(exl3o_f32_to_bf16(v));
            if (bias) v = x_dtype == DT_F16 ? rh(v + h2f(bias[n])) : v + h2f(bias[n]);
            store_y(y, y_dtype, m * out + n, v);
        }
    }
done:
    free(xin);
    free(yh);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* MoE SwitchGLU                                                             */
/* ------------------------------------------------------------------------ */

/* Inner product of one input row against the tile columns [col_tile0,
 * col_tile0 + width/16) of a trellis with tn_total tile columns. */
static void expert_gemv(const float* xin, const uint16_t* trellis, int in, int tn_total,
                        int col_tile0, int width, int k, const uint16_t* table,
                        const uint16_t* perm, float* yh) {
    for (int c = 0; c < width; ++c) yh[c] = 0.0f;
    float w[256];
    uint16_t st[256];
    for (int tn = 0; tn < width / 16; ++tn)
        for (int tk = 0; tk < in / 16; ++tk) {
            unpack_tile(trellis + ((int64_t)tk * tn_total + col_tile0 + tn) * 16 * k, k, st);
            for (int i = 0; i < 256; ++i) w[perm[i]] = h2f(table[st[i]]);
            for (int r = 0; r < 16; ++r) {
                float xv = xin[tk * 16 + r];
                for (int c = 0; c < 16; ++c) yh[tn * 16 + c] += xv * w[r * 16 + c];
            }
        }
}

/* expert_mapped (linear.rs:2817-2852; expert_mapped_layout :3054-3336 for a
 * route-major bank, the MLX path): row r = route * projections + p of x
 * [rows][in] gets xhat = f16(x) * suh[r] (f16) -> MLX f16 H128 (the prologue
 * of exl3o_prologue with the row's scales), times the bank's tile columns
 * selected[route] * out/16 + p * stride_tiles + t (t < out/16) in f32
 * (expert_gemv); raw: y f32 = that product; else f16(yhat) -> f16 H128 ->
 * * svh[r] (f16) -> x's dtype (the linear's mode-1 epilogue without bias).
 * Rows whose columns leave the bank are zero (the HIP build's choice for
 * device-side expert indices the reference does not check). */
int exl3o_expert_mapped(const void* x, int x_dtype, int64_t rows, int in, const uint16_t* suh,
                        const uint16_t* trellis, int bank_tiles, int k, int cb,
                        const uint32_t* selected, int routes, int projections, int out,
                        int stride_tiles, const uint16_t* svh, int raw, void* y, int threads) {
    if (!valid_dtype(x_dtype) || k < 1 || k > 8 || k == 7 || cb < 0 || cb > 2) return -1;
    if (in <= 0 || in % 128 || out <= 0 || out % 128 || bank_tiles <= 0) return -1;
    if (projections <= 0 || routes <= 0 || (int64_t)routes * projections != rows) return -1;
    if (stride_tiles < 0 || (int64_t)(projections - 1) * stride_tiles + out / 16 > bank_tiles)
        return -1;
    if (!x || !suh || !trellis || !selected || !y || (!raw && !svh)) return -1;
    const uint16_t* table = codebook_table(cb);
    if (!table) return -3;
    uint16_t perm[256];
    exl3o_permutation(perm);
    const size_t xsz = x_dtype == DT_F32 ? 4 : 2;
    int err = 0;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#else
    (void)threads;
#endif
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int64_t r = 0; r < rows; ++r) {
        uint16_t* xhat = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)in);
        float* xin = (float*)malloc(sizeof(float) * (size_t)in);
        float* yh = (float*)malloc(sizeof(float) * (size_t)out);
        if (!xhat || !xin || !yh) {
#pragma omp atomic write
            err = -3;
        } else {
            exl3o_prologue((const char*)x + (size_t)r * in * xsz, x_dtype, 1, in,
                           suh + (size_t)r * in, xhat);
            for (int i = 0; i < in; ++i) xin[i] = h2f(xhat[i]);
            const int64_t route = r / projections, p = r - route * projections;
            const int64_t base = (int64_t)selected[route] * (out / 16) + p * stride_tiles;
            if (base + out / 16 <= bank_tiles)
                expert_gemv(xin, trellis, in, bank_tiles, (int)base, out, k, table, perm, yh);
            else
                for (int n = 0; n < out; ++n) yh[n] = 0.0f;
            if (raw) {
                memcpy((float*)y + (size_t)r * out, yh, sizeof(float) * (size_t)out);
            } else {
                for (int n = 0; n < out; ++n) yh[n] = rh(yh[n]);
                exl3o_h128_staged(yh, out);
                for (int n = 0; n < out; ++n) {
                    float v = rh(yh[n] * h2f(svh[(size_t)r * out + n]));
                    if (x_dtype == DT_BF16) v = exl3o_bf16_to_f32(exl3o_f32_to_bf16(v));
                    store_y(y, x_dtype, r * out + n, v);
                }
            }
        }
        free(xhat);
        free(xin);
        free(yh);
    }
    return err;
}

/* Exl3SwitchGlu::forward (moe.rs:905-975) for SiLU: routed_inputs
 * (moe.rs:184-250: f16(x*suh), MLX f16 H128 schedule), expert QMM raw outputs,
 * glu_down_input (moe.rs:435-563: f16(raw) -> f32 H128 -> f16(v*s*svh),
 * f16(silu(g)*u), f16(a*down_suh), f32 H128, f16(v*s)), then finish_and_reduce
 * (moe.rs:586-609: f16(raw) -> MLX f16 H128 -> *svh (f16) -> *score (f16) ->
 * f32 sum over top-k -> f16). */
/* One element of Array::geglu (native/ffi/mlx_bridge.cpp:764-774): the
 * compiled MLX expression 0.5g * (1 + tanh(0.7978845608 * (g + 0.044715 g^3)))
 * * u on float16 arrays.  Every operation rounds to f16 (the constants are
 * f16 scalars); pow(g, 3) and tanh are rounded once from binary64 (g^3 is
 * exact there). */
static float geglu1(float g, float u) {
    const double gd = g;
    const float cube = h2f(exl3o_f64_to_f16(gd * gd * gd));
    const float t = rh(g + rh(rh(0.044715f) * cube));
    const float inner = rh(rh(0.7978845608028654f) * t);
    const float th = h2f(exl3o_f64_to_f16(tanh((double)inner)));
    const float gelu = rh(rh(0.5f * g) * rh(1.0f + th));
    return rh(gelu * u);
}

void exl3o_geglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f2h(geglu1(h2f(gate[i]), h2f(up[i])));
}

int exl3o_moe_forward(const void* x, int x_dtype, int64_t rows, int in, int hidden, int experts,
                      int top_k, int k, int cb, const uint16_t* gu_trellis,
                      const uint16_t* gu_suh, const uint16_t* gu_svh,
                      const uint16_t* down_trellis, const uint16_t* down_suh,
                      const uint16_t* down_svh, const uint32_t* selected, const void* scores,
                      int scores_dtype, void* y, int gelu, int logical_hidden, int threads) {
    if (k < 1 || k > 8 || cb < 0 || cb > 2 || rows < 1 || top_k < 1 || experts < 1) return -1;
    if (!valid_dtype(x_dtype) || !valid_dtype(scores_dtype)) return -1;
    if (in % 128 || hidden % 128 || in <= 0 || hidden <= 0) return -1;
    if (gelu && logical_hidden <= 0) return -1; /* >= hidden: nothing is zeroed */
    for (int64_t i = 0; i < rows * top_k; ++i)
        if (selected[i] >= (uint32_t)experts) return -1;
    const uint16_t* table = codebook_table(cb);
    if (!table) return -3;
    uint16_t perm[256];
    exl3o_permutation(perm);
    const float s = had_scale();
    const int gu_tn = 2 * experts * hidden / 16, down_tn = experts * in / 16;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#else
    (void)threads;
#endif
    int err = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (int64_t r = 0; r < rows; ++r) {
        int big = in > hidden ? in : hidden;
        float* xin = (float*)malloc(sizeof(float) * (size_t)big);
        float* g = (float*)malloc(sizeof(float) * (size_t)hidden);
        float* u = (float*)malloc(sizeof(float) * (size_t)hidden);
        float* d = (float*)malloc(sizeof(float) * (size_t)in);
        float* sum = (float*)calloc((size_t)in, sizeof(float));
        if (!xin || !g || !u || !d || !sum) {
#pragma omp atomic write
            err = -3;
            free(xin), free(g), free(u), free(d), free(sum);
            continue;
        }
        for (int t = 0; t < top_k; ++t) {
            uint32_t e = selected[r * top_k + t];
            for (int p = 0; p < 2; ++p) {
                const uint16_t* su = gu_suh + ((size_t)e * 2 + p) * in;
                /* routed_inputs (moe.rs:205-206): half(half(x) * half(scale)) */
                for (int i = 0; i < in; ++i)
                    xin[i] = rh(rh(load_x(x, x_dtype, r * in + i)) * h2f(su[i]));
                exl3o_h128_staged(xin, in);
                expert_gemv(xin, gu_trellis, in, gu_tn, (int)((p * experts + e) * hidden / 16),
                            hidden, k, table, perm, p ? u : g);
            }
            const uint16_t* dsu = down_suh + (size_t)e * hidden;
            if (gelu) {
                /* forward_gelu (moe.rs:1087-1153): gate and up as expert_mapped
                 * returns them (linear.rs:3325-3331: f16, staged H128, *svh in
                 * f16), GEGLU, zeros from logical_hidden on, and the down input
                 * as expert_mapped prepares it (linear.rs:3131-3137). */
                for (int p = 0; p < 2; ++p) {
                    float* v = p ? u : g;
                    const uint16_t* sv = gu_svh + ((size_t)e * 2 + p) * hidden;
                    for (int i = 0; i < hidden; ++i) v[i] = rh(v[i]);
                    exl3o_h128_staged(v, hidden);
                    for (int i = 0; i < hidden; ++i) v[i] = rh(v[i] * h2f(sv[i]));
                }
                for (int i = 0; i < hidden; ++i) {
                    const float act = i < logical_hidden ? geglu1(g[i], u[i]) : 0.0f;
                    xin[i] = rh(act * h2f(dsu[i]));
                }
                exl3o_h128_staged(xin, hidden);
            } else {
                /* glu_down_input (moe.rs:435-563), SiLU */
                for (int p = 0; p < 2; ++p) {
                    float* v = p ? u : g;
                    const uint16_t* sv = gu_svh + ((size_t)e * 2 + p) * hidden;
                    for (int i = 0; i < hidden; ++i) v[i] = rh(v[i]);
                    for (int b = 0; b < hidden; b += 128)
                        for (int stride = 1; stride < 128; stride <<= 1)
                            butterfly_stage(v + b, stride);
                    for (int i = 0; i < hidden; ++i) v[i] = rh(v[i] * s * h2f(sv[i]));
                }
                for (int i = 0; i < hidden; ++i) {
                    float gv = g[i], uv = u[i];
                    float act = rh((gv / (1.0f + expf(-gv))) * uv);
                    xin[i] = rh(act * h2f(dsu[i]));
                }
                for (int b = 0; b < hidden; b += 128)
                    for (int stride = 1; stride < 128; stride <<= 1)
                        butterfly_stage(xin + b, stride);
                for (int i = 0; i < hidden; ++i) xin[i] = rh(xin[i] * s);
            }
            expert_gemv(xin, down_trellis, hidden, down_tn, (int)(e * in / 16), in, k, table, perm,
                        d);
            for (int i = 0; i < in; ++i) d[i] = rh(d[i]);
            exl3o_h128_staged(d, in);
            const uint16_t* dsv = down_svh + (size_t)e * in;
            const float sc = load_score(scores, scores_dtype, r * top_k + t);
            for (int i = 0; i < in; ++i) sum[i] += weighted(rh(d[i] * h2f(dsv[i])), sc, scores_dtype);
        }
        for (int i = 0; i < in; ++i) store_reduced(y, scores_dtype, r * in + i, sum[i]);
        free(xin), free(g), free(u), free(d), free(sum);
    }
    return err;
}

/* glu_down_input, SiLU (moe.rs:435-563, swiglu_down_input :569-583): per slot
 * s and 128-column block, gate = f16(raw[2s]) and up = f16(raw[2s+1]) through
 * an f32 H128 and f16(v * scale * svh[e][p]), act = f16(silu(gate) * up),
 * f16(act * down_suh[e]), an f32 H128 and f16(v * scale). */
int exl3o_swiglu_down_input(const float* gate_up, const uint16_t* gu_svh,
                            const uint16_t* down_suh, const uint32_t* selected, int64_t slots,
                            int hidden, int experts, uint16_t* xhat) {
    if (slots < 1 || hidden <= 0 || hidden % 128 || experts < 1) return -1;
    for (int64_t i = 0; i < slots; ++i)
        if (selected[i] >= (uint32_t)experts) return -1;
    const float s = had_scale();
    float g[128], u[128], d[128];
    for (int64_t sl = 0; sl < slots; ++sl) {
        const uint32_t e = selected[sl];
        for (int b = 0; b < hidden; b += 128) {
            for (int i = 0; i < 128; ++i) {
                g[i] = rh(gate_up[(2 * sl) * hidden + b + i]);
                u[i] = rh(gate_up[(2 * sl + 1) * hidden + b + i]);
            }
            for (int stride = 1; stride < 128; stride <<= 1) {
                butterfly_stage(g, stride);
                butterfly_stage(u, stride);
            }
            for (int i = 0; i < 128; ++i) {
                const float gv = rh(g[i] * s * h2f(gu_svh[((size_t)e * 2) * hidden + b + i]));
                const float uv = rh(u[i] * s * h2f(gu_svh[((size_t)e * 2 + 1) * hidden + b + i]));
                const float act = rh((gv / (1.0f + expf(-gv))) * uv);
                d[i] = rh(act * h2f(down_suh[(size_t)e * hidden + b + i]));
            }
            for (int stride = 1; stride < 128; stride <<= 1) butterfly_stage(d, stride);
            for (int i = 0; i < 128; ++i) xhat[sl * hidden + b + i] = f2h(d[i] * s);
        }
    }
    return 0;
}

/* finish_and_reduce (moe.rs:586-609): y[r] = sum_t weighted(f16(f16(H(f16(raw)))
 * * svh), score) over the top_k slots r*top_k + t in f32 (f16 result for f16
 * scores), H the staged H128 with f16(v * scale). */
int exl3o_finish_and_reduce(const float* raw, const uint16_t* svh, const void* scores,
                            int scores_dtype, int64_t rows, int top_k, int width, void* y) {
    if (rows < 1 || top_k < 1 || width <= 0 || width % 128) return -1;
    if (!valid_dtype(scores_dtype)) return -1;
    float* v = (float*)malloc(sizeof(float) * (size_t)width);
    float* acc = (float*)malloc(sizeof(float) * (size_t)width);
    if (!v || !acc) {
        free(v), free(acc);
        return -3;
    }
    for (int64_t r = 0; r < rows; ++r) {
        for (int i = 0; i < width; ++i) acc[i] = 0.0f;
        for (int t = 0; t < top_k; ++t) {
            const int64_t sl = r * top_k + t;
            for (int i = 0; i < width; ++i) v[i] = rh(raw[sl * width + i]);
            exl3o_h128_staged(v, width);
            const float sc = load_score(scores, scores_dtype, sl);
            for (int i = 0; i < width; ++i)
                acc[i] += weighted(rh(v[i] * h2f(svh[sl * width + i])), sc, scores_dtype);
        }
        for (int i = 0; i < width; ++i) store_reduced(y, scores_dtype, r * width + i, acc[i]);
    }
    free(v), free(acc);
    return 0;
}

/* ---- dense SwiGLU: mlx_bridge.cpp:745-749 (MLX Sigmoid on float16) ---- */
void exl3o_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = h2f(gate[i]), u = h2f(up[i]);
        const float e = rh(expf(-fabsf(g)));
        const float y = rh(1.0f / rh(1.0f + e));
        const float s = g < 0.0f ? rh(1.0f - y) : y;
        out[i] = f2h(rh(g * s) * u);
    }
}
