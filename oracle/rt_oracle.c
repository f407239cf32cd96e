/*
 * rt_oracle.c -- CPU restatement of rich-triplet's quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See rt_oracle.h
 * for what pins each function.  Build: oracle/Makefile, with
 * -ffp-contract=off -fno-fast-math so every f32 operation rounds exactly where
 * the reference's does.
 */
#include "rt_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define Q4K_SUPERBLOCK 256u
#define Q4K_BLOCK_BYTES 144u

/* ------------------------------------------------------------------------ */
/* bit casts                                                                */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------------ */
/* include/rt/bf16.hpp:42-126                                               */
/* ------------------------------------------------------------------------ */

float orc_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

uint16_t orc_f32_to_bf16(float v) {
    const uint32_t bits = f2u(v);
    if (isnan(v)) {
        return (uint16_t)((bits >> 16) | 0x0040u);
    }
    const uint32_t bias = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((uint32_t)(bits + bias) >> 16);
}

float orc_f16_to_f32(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t exp = (bits >> 10) & 0x1fu;
    const uint32_t mant = bits & 0x3ffu;
    if (exp == 0) {
        if (mant == 0) return u2f(sign);
        /* subnormal: shift until the implicit one appears */
        uint32_t m = mant, e = 0;
        while ((m & 0x400u) == 0) {
            m <<= 1;
            ++e;
        }
        m &= 0x3ffu;
        return u2f(sign | ((127u - 15u - e + 1u) << 23) | (m << 13));
    }
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15u + 127u) << 23) | (mant << 13));
}

uint16_t orc_f32_to_f16(float v) {
    /* truncating conversion (the mantissa is cut, never rounded) */
    const uint32_t bits = f2u(v);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant >> 13));
    const int32_t e16 = exp - 127 + 15;
    if (e16 >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e16 <= 0) {
        if (e16 < -10) return (uint16_t)sign;
        const uint32_t m = mant | 0x800000u;
        const uint32_t shift = (uint32_t)(1 - e16) + 13u;
        return (uint16_t)(sign | (m >> shift));
    }
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | (mant >> 13));
}

void orc_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}

/* ------------------------------------------------------------------------ */
/* threading: include/rt/parallel.hpp:18-42                                 */
/* ------------------------------------------------------------------------ */

int orc_hardware_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n <= 0 ? 1 : (int)n;
}

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

typedef void (*band_fn)(void* ctx, size_t tid);
struct spawn_arg {
    band_fn fn;
    void* ctx;
    size_t tid;
};
static void* spawn_trampoline(void* p) {
    struct spawn_arg* a = (struct spawn_arg*)p;
    a->fn(a->ctx, a->tid);
    return NULL;
}
/* scoped_spawn: inline when n <= 1, else n threads joined before return */
static void scoped_spawn(size_t n, band_fn fn, void* ctx) {
    if (n <= 1) {
        fn(ctx, 0);
        return;
    }
    pthread_t* th = (pthread_t*)malloc(n * sizeof(pthread_t));
    struct spawn_arg* args = (struct spawn_arg*)malloc(n * sizeof(struct spawn_arg));
    for (size_t t = 0; t < n; ++t) {
        args[t].fn = fn;
        args[t].ctx = ctx;
        args[t].tid = t;
        pthread_create(&th[t], NULL, spawn_trampoline, &args[t]);
    }
    for (size_t t = 0; t < n; ++t) pthread_join(th[t], NULL);
    free(args);
    free(th);
}

/* ------------------------------------------------------------------------ */
/* Q4_K: src/quant_q4k.cpp                                                  */
/* ------------------------------------------------------------------------ */

uint8_t orc_sat_u8(float v) {
    if (!(v > 0.0f)) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}

static inline uint8_t min_u8(uint8_t a, uint8_t b) { return b < a ? b : a; }
static inline float std_min(float a, float b) { return b < a ? b : a; } /* std::min */
static inline float std_max(float a, float b) { return a < b ? b : a; } /* std::max */
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void orc_q4k_pack_scales(const uint8_t sv[8], const uint8_t mv[8], uint8_t sc[12]) {
    for (size_t j = 0; j < 4; ++j) {
        sc[j] = (uint8_t)((sv[j] & 0x3f) | ((sv[j + 4] & 0x30) << 2));
        sc[j + 4] = (uint8_t)((mv[j] & 0x3f) | ((mv[j + 4] & 0x30) << 2));
    }
    for (size_t j = 0; j < 4; ++j) {
        sc[8 + j] = (uint8_t)((sv[j + 4] & 0x0f) | ((mv[j + 4] & 0x0f) << 4));
    }
}

void orc_q4k_scale_min(const uint8_t* sc, size_t j, float* scale, float* min) {
    uint8_t sv, mv;
    if (j < 4) {
        sv = sc[j] & 0x3f;
        mv = sc[j + 4] & 0x3f;
    } else {
        sv = (uint8_t)((sc[j + 4] & 0x0f) | ((sc[j - 4] >> 6) << 4));
        mv = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
    *scale = (float)sv;
    *min = (float)mv;
}

void orc_q4k_quantize_block(const float* x, uint8_t* out) {
    float sub_scales[8] = {0}, sub_mins[8] = {0};
    for (size_t sb = 0; sb < 8; ++sb) {
        const float* s = x + sb * 32;
        float smin = INFINITY, smax = -INFINITY;
        for (size_t i = 0; i < 32; ++i) {
            smin = std_min(smin, s[i]);
            smax = std_max(smax, s[i]);
        }
        if (smin >= 0.0f) {
            sub_mins[sb] = 0.0f;
            sub_scales[sb] = smax > 0.0f ? smax / 15.0f : 0.0f;
        } else {
            sub_mins[sb] = smin;
            sub_scales[sb] = smax > smin ? (smax - smin) / 15.0f : 0.0f;
        }
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (size_t j = 0; j < 8; ++j) {
        max_scale = std_max(max_scale, sub_scales[j]);
        max_min = std_max(max_min, -sub_mins[j]);
    }
    const float d = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    const float dmin = max_min > 0.0f ? max_min / 63.0f : 0.0f;

    uint8_t sv[8] = {0}, mv[8] = {0};
    if (d > 0.0f) {
        const float inv = 1.0f / d;
        for (size_t j = 0; j < 8; ++j) sv[j] = min_u8(63, orc_sat_u8(sub_scales[j] * inv + 0.5f));
    }
    if (dmin > 0.0f) {
        const float inv = 1.0f / dmin;
        for (size_t j = 0; j < 8; ++j) mv[j] = min_u8(63, orc_sat_u8(-sub_mins[j] * inv + 0.5f));
    }
    const uint16_t d16 = orc_f32_to_f16(d), m16 = orc_f32_to_f16(dmin);
    out[0] = (uint8_t)(d16 & 0xff);
    out[1] = (uint8_t)(d16 >> 8);
    out[2] = (uint8_t)(m16 & 0xff);
    out[3] = (uint8_t)(m16 >> 8);
    orc_q4k_pack_scales(sv, mv, out + 4);

    const float dv = orc_f16_to_f32(d16), mvv = orc_f16_to_f32(m16);
    for (size_t c = 0; c < 4; ++c) {
        const float s1 = dv * (float)sv[2 * c], n1 = mvv * (float)mv[2 * c];
        const float s2 = dv * (float)sv[2 * c + 1], n2 = mvv * (float)mv[2 * c + 1];
        const float* lo = x + c * 64;
        const float* hi = lo + 32;
        for (size_t l = 0; l < 32; ++l) {
            const uint8_t ql = s1 > 0.0f ? min_u8(15, orc_sat_u8((lo[l] + n1) / s1 + 0.5f)) : 0;
            const uint8_t qh = s2 > 0.0f ? min_u8(15, orc_sat_u8((hi[l] + n2) / s2 + 0.5f)) : 0;
            out[16 + c * 32 + l] = (uint8_t)(ql | (qh << 4));
        }
    }
}

struct q4k_build_ctx {
    const float* wf;
    const uint16_t* wb;
    size_t rows, cols, per_thread;
    uint8_t* blocks;
};

static void q4k_build_band(void* p, size_t tid) {
    struct q4k_build_ctx* c = (struct q4k_build_ctx*)p;
    const size_t r0 = tid * c->per_thread;
    if (r0 >= c->rows) return;
    const size_t r1 = r0 + c->per_thread < c->rows ? r0 + c->per_thread : c->rows;
    const size_t nb = c->cols / Q4K_SUPERBLOCK;
    float* buf = (float*)malloc(c->cols * sizeof(float));
    for (size_t r = r0; r < r1; ++r) {
        if (c->wf) {
            memcpy(buf, c->wf + r * c->cols, c->cols * sizeof(float));
        } else {
            for (size_t i = 0; i < c->cols; ++i) buf[i] = orc_bf16_to_f32(c->wb[r * c->cols + i]);
        }
        for (size_t b = 0; b < nb; ++b)
            orc_q4k_quantize_block(buf + b * Q4K_SUPERBLOCK,
                                   c->blocks + (r * nb + b) * Q4K_BLOCK_BYTES);
    }
    free(buf);
}

static void q4k_build(const float* wf, const uint16_t* wb, size_t rows, size_t cols,
                      uint8_t* blocks, int n_threads) {
    const size_t nt = n_threads < 1 ? 1 : (size_t)n_threads;
    struct q4k_build_ctx c = {wf, wb, rows, cols, div_ceil(rows, nt), blocks};
    memset(blocks, 0, rows * (cols / Q4K_SUPERBLOCK) * Q4K_BLOCK_BYTES);
    scoped_spawn(nt, q4k_build_band, &c);
}

void orc_q4k_quantize(const float* w, size_t rows, size_t cols, uint8_t* blocks,
                      int n_threads) {
    q4k_build(w, NULL, rows, cols, blocks, n_threads);
}

void orc_q4k_quantize_from_bf16(const uint16_t* w, size_t rows, size_t cols, uint8_t* blocks,
                                int n_threads) {
    q4k_build(NULL, w, rows, cols, blocks, n_threads);
}

void orc_q4k_dequant_row(const uint8_t* blocks, size_t cols, size_t row, float* out) {
    const size_t nb = cols / Q4K_SUPERBLOCK;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* bp = blocks + (row * nb + b) * Q4K_BLOCK_BYTES;
        const float d = orc_f16_to_f32(rd16(bp)), dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t* sc = bp + 4;
        const uint8_t* qs = bp + 16;
        float* o = out + b * Q4K_SUPERBLOCK;
        for (size_t c = 0; c < 4; ++c) {
            float sv1, mv1, sv2, mv2;
            orc_q4k_scale_min(sc, 2 * c, &sv1, &mv1);
            orc_q4k_scale_min(sc, 2 * c + 1, &sv2, &mv2);
            const float s1 = d * sv1, n1 = dmin * mv1, s2 = d * sv2, n2 = dmin * mv2;
            const uint8_t* q = qs + c * 32;
            for (size_t l = 0; l < 32; ++l) {
                o[c * 64 + l] = s1 * (float)(q[l] & 0x0f) - n1;
                o[c * 64 + 32 + l] = s2 * (float)(q[l] >> 4) - n2;
            }
        }
    }
}

float orc_q4k_dot_row(const uint8_t* blocks, size_t cols, size_t row, const float* a) {
    const size_t nb = cols / Q4K_SUPERBLOCK;
    float acc = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* bp = blocks + (row * nb + b) * Q4K_BLOCK_BYTES;
        const float d = orc_f16_to_f32(rd16(bp)), dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t* sc = bp + 4;
        const uint8_t* qs = bp + 16;
        for (size_t c = 0; c < 4; ++c) {
            float sv1, mv1, sv2, mv2;
            orc_q4k_scale_min(sc, 2 * c, &sv1, &mv1);
            orc_q4k_scale_min(sc, 2 * c + 1, &sv2, &mv2);
            const float s1 = d * sv1, n1 = dmin * mv1, s2 = d * sv2, n2 = dmin * mv2;
            const uint8_t* q = qs + c * 32;
            const size_t off = b * Q4K_SUPERBLOCK + c * 64;
            float dot_lo = 0.0f, dot_hi = 0.0f, sum_lo = 0.0f, sum_hi = 0.0f;
            for (size_t l = 0; l < 32; ++l) {
                const float alo = a[off + l];
                dot_lo += (float)(q[l] & 0x0f) * alo;
                sum_lo += alo;
                const float ahi = a[off + 32 + l];
                dot_hi += (float)(q[l] >> 4) * ahi;
                sum_hi += ahi;
            }
            acc += s1 * dot_lo - n1 * sum_lo + s2 * dot_hi - n2 * sum_hi;
        }
    }
    return acc;
}

struct gemv_ctx {
    const uint8_t* q4k;
    const uint16_t* bf16;
    size_t rows, cols, chunk;
    const float* a;
    float* y;
};

static void q4k_gemv_band(void* p, size_t tid) {
    struct gemv_ctx* c = (struct gemv_ctx*)p;
    const size_t j0 = tid * c->chunk;
    if (j0 >= c->rows) return;
    const size_t j1 = j0 + c->chunk < c->rows ? j0 + c->chunk : c->rows;
    for (size_t j = j0; j < j1; ++j) c->y[j] = orc_q4k_dot_row(c->q4k, c->cols, j, c->a);
}

static size_t gemv_threads(int n_threads, size_t rows) {
    size_t hw = n_threads < 1 ? 1 : (size_t)n_threads;
    size_t t = rows / 128 < hw ? rows / 128 : hw;
    return t < 1 ? 1 : t;
}

void orc_q4k_gemv_mt(const uint8_t* blocks, size_t rows, size_t cols, const float* a,
                     float* y, int n_threads) {
    const size_t nt = gemv_threads(n_threads, rows);
    struct gemv_ctx c = {blocks, NULL, rows, cols, div_ceil(rows, nt), a, y};
    memset(y, 0, rows * sizeof(float));
    scoped_spawn(nt, q4k_gemv_band, &c);
}

void orc_q4k_matmul_t(const uint8_t* blocks, size_t rows, size_t cols, const float* a,
                      size_t m, float* y, int n_threads, size_t r0, size_t r1) {
    if (m == 1 && r0 == 0 && r1 == rows) {
        orc_q4k_gemv_mt(blocks, rows, cols, a, y, n_threads);
        return;
    }
    if (m == 1) { /* row slice of the M == 1 path: same dot_row per row */
        for (size_t j = r0; j < r1; ++j) y[j] = orc_q4k_dot_row(blocks, cols, j, a);
        return;
    }
    /* zero-initialised row buffer: with cols % 256 != 0 its tail stays 0 */
    float* buf = (float*)calloc(cols, sizeof(float));
    for (size_t j = r0; j < r1; ++j) {
        orc_q4k_dequant_row(blocks, cols, j, buf);
        for (size_t i = 0; i < m; ++i) {
            float acc = 0.0f;
            for (size_t p = 0; p < cols; ++p) acc += a[i * cols + p] * buf[p];
            y[i * rows + j] = acc;
        }
    }
    free(buf);
}

void orc_q4k_quantize_activation_q8(const float* a, size_t k, int8_t* q8, float* scales,
                                    float* sums) {
    const size_t nb = div_ceil(k, 32);
    memset(q8, 0, nb * 32);
    for (size_t blk = 0; blk < nb; ++blk) {
        const size_t s = blk * 32, e = s + 32 < k ? s + 32 : k;
        float max_abs = 0.0f, sum = 0.0f;
        for (size_t i = s; i < e; ++i) {
            max_abs = std_max(max_abs, fabsf(a[i]));
            sum += a[i];
        }
        sums[blk] = sum;
        if (max_abs == 0.0f) {
            scales[blk] = 0.0f;
            continue;
        }
        const float scale = max_abs / 127.0f;
        const float inv = 1.0f / scale;
        scales[blk] = scale;
        for (size_t i = s; i < e; ++i) {
            float r = roundf(a[i] * inv);
            r = r < -128.0f ? -128.0f : (127.0f < r ? 127.0f : r);
            q8[i] = (int8_t)r;
        }
    }
}

/* dot_row_q8 (src/quant_q4k.cpp:425-478, the aarch64 SDOT branch): per
 * 64-value chunk of a super-block, the exact integer dots of the low nibbles
 * with q8[64c .. 64c+32) and of the high nibbles with q8[64c+32 .. 64c+64)
 * (vdotq_s32 lanes summed: an exact int32), then
 *     total += d*sv1*scale_lo*idot_lo - dmin*mv1*sum_lo
 *            + d*sv2*scale_hi*idot_hi - dmin*mv2*sum_hi
 * left to right, each operation rounded (the reference builds with
 * -ffp-contract=off, CMakeLists.txt:17-47).  The NEON intrinsics do not
 * compile here; the integer dot is written as the plain sum it computes. */
float orc_q4k_dot_row_q8(const uint8_t* blocks, size_t cols, size_t row, const int8_t* q8,
                         const float* scales, const float* sums) {
    const size_t nb = cols / Q4K_SUPERBLOCK;
    float total = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* bp = blocks + (row * nb + b) * Q4K_BLOCK_BYTES;
        const float d = orc_f16_to_f32(rd16(bp)), dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t* sc = bp + 4;
        const uint8_t* qs = bp + 16;
        const size_t a_base = b * Q4K_SUPERBLOCK;
        for (size_t c = 0; c < 4; ++c) {
            float sv1, mv1, sv2, mv2;
            orc_q4k_scale_min(sc, 2 * c, &sv1, &mv1);
            orc_q4k_scale_min(sc, 2 * c + 1, &sv2, &mv2);
            const uint8_t* q = qs + c * 32;
            const size_t lo = a_base + c * 64, hi = lo + 32;
            int32_t idot_lo = 0, idot_hi = 0;
            for (size_t l = 0; l < 32; ++l) {
                idot_lo += (int32_t)(q[l] & 0x0f) * (int32_t)q8[lo + l];
                idot_hi += (int32_t)(q[l] >> 4) * (int32_t)q8[hi + l];
            }
            total += d * sv1 * scales[lo / 32] * (float)idot_lo - dmin * mv1 * sums[lo / 32] +
                     d * sv2 * scales[hi / 32] * (float)idot_hi - dmin * mv2 * sums[hi / 32];
        }
    }
    return total;
}

/* gemv_mt's aarch64 branch (src/quant_q4k.cpp:564-600): the activation is
 * quantized once (quantize_activation_q8), then every row takes dot_row_q8.
 * Rows are independent, so one thread computes them all here. */
void orc_q4k_gemv_q8(const uint8_t* blocks, size_t rows, size_t cols, const float* a, float* y) {
    const size_t nb32 = div_ceil(cols, 32);
    int8_t* q8 = (int8_t*)calloc(nb32 * 32, 1);
    float* sc = (float*)calloc(nb32, sizeof(float));
    float* su = (float*)calloc(nb32, sizeof(float));
    orc_q4k_quantize_activation_q8(a, cols, q8, sc, su);
    for (size_t j = 0; j < rows; ++j) y[j] = orc_q4k_dot_row_q8(blocks, cols, j, q8, sc, su);
    free(q8);
    free(sc);
    free(su);
}

/* ------------------------------------------------------------------------ */
/* BF16: src/mat.cpp:304-414                                                 */
/* ------------------------------------------------------------------------ */

float orc_bf16_dot_row(const uint16_t* w, size_t cols, size_t row, const float* a) {
    const uint16_t* r = w + row * cols;
    float acc = 0.0f;
    for (size_t p = 0; p < cols; ++p) acc += orc_bf16_to_f32(r[p]) * a[p];
    return acc;
}

static void bf16_gemv_band(void* p, size_t tid) {
    struct gemv_ctx* c = (struct gemv_ctx*)p;
    const size_t j0 = tid * c->chunk;
    if (j0 >= c->rows) return;
    const size_t j1 = j0 + c->chunk < c->rows ? j0 + c->chunk : c->rows;
    for (size_t j = j0; j < j1; ++j) c->y[j] = orc_bf16_dot_row(c->bf16, c->cols, j, c->a);
}

void orc_bf16_gemv_mt(const uint16_t* w, size_t rows, size_t cols, const float* a, float* y,
                      int n_threads) {
    const size_t nt = gemv_threads(n_threads, rows);
    struct gemv_ctx c = {NULL, w, rows, cols, div_ceil(rows, nt), a, y};
    memset(y, 0, rows * sizeof(float));
    scoped_spawn(nt, bf16_gemv_band, &c);
}

void orc_bf16_matmul_t(const uint16_t* w, size_t rows, size_t cols, const float* a, size_t m,
                       float* y, int n_threads, size_t r0, size_t r1) {
    if (m == 1 && r0 == 0 && r1 == rows) {
        orc_bf16_gemv_mt(w, rows, cols, a, y, n_threads);
        return;
    }
    if (m == 1) {
        for (size_t j = r0; j < r1; ++j) y[j] = orc_bf16_dot_row(w, cols, j, a);
        return;
    }
    float* buf = (float*)malloc(cols * sizeof(float));
    for (size_t j = r0; j < r1; ++j) {
        for (size_t c = 0; c < cols; ++c) buf[c] = orc_bf16_to_f32(w[j * cols + c]);
        for (size_t i = 0; i < m; ++i) {
            float dot = 0.0f;
            for (size_t c = 0; c < cols; ++c) dot += a[i * cols + c] * buf[c];
            y[i * rows + j] = dot;
        }
    }
    free(buf);
}

/* ------------------------------------------------------------------------ */
/* Q4Mat: src/quant_q4.cpp:17-114                                            */
/* ------------------------------------------------------------------------ */

void orc_q4mat_quantize(const float* w, size_t n, uint8_t* packed, float* scales) {
    const size_t nblk = div_ceil(n, 32);
    memset(packed, 0, div_ceil(n, 2));
    for (size_t blk = 0; blk < nblk; ++blk) {
        const size_t s = blk * 32, e = s + 32 < n ? s + 32 : n;
        float absmax = 0.0f;
        for (size_t k = s; k < e; ++k) absmax = std_max(absmax, fabsf(w[k]));
        const float scale = absmax == 0.0f ? 1.0f : absmax / 7.0f;
        scales[blk] = scale;
        for (size_t k = s; k < e; ++k) {
            float r = roundf(w[k] / scale);
            r = r < -7.0f ? -7.0f : (7.0f < r ? 7.0f : r);
            const uint8_t nib = (uint8_t)((int8_t)r & 0x0f);
            if (k % 2 == 0)
                packed[k / 2] |= nib;
            else
                packed[k / 2] |= (uint8_t)(nib << 4);
        }
    }
}

static inline int q4_nibble(const uint8_t* packed, size_t k) {
    const int nib = (k % 2 == 0) ? (packed[k / 2] & 0x0f) : ((packed[k / 2] >> 4) & 0x0f);
    return nib >= 8 ? nib - 16 : nib;
}

void orc_q4mat_dequant(const uint8_t* packed, const float* scales, size_t n, float* out) {
    for (size_t k = 0; k < n; ++k) out[k] = (float)q4_nibble(packed, k) * scales[k / 32];
}

void orc_q4mat_matmul_t(const uint8_t* packed, const float* scales, size_t rows, size_t cols,
                        const float* a, size_t m, float* y) {
    for (size_t j = 0; j < rows; ++j) {
        const size_t base = j * cols;
        for (size_t i = 0; i < m; ++i) {
            float acc = 0.0f;
            for (size_t p = 0; p < cols; ++p) {
                const size_t f = base + p;
                const float w = (float)q4_nibble(packed, f) * scales[f / 32];
                acc += a[i * cols + p] * w;
            }
            y[i * rows + j] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GGUF Q4_0 and Q6_K: src/gguf.cpp                                         */
/* ------------------------------------------------------------------------ */

void orc_q4_0_decode_f32(const uint8_t* blocks, size_t n_elem, float* out) {
    const size_t nb = div_ceil(n_elem, 32);
    memset(out, 0, n_elem * sizeof(float));
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* bp = blocks + b * 18;
        const float scale = orc_f16_to_f32(rd16(bp));
        const size_t s = b * 32, e = s + 32 < n_elem ? s + 32 : n_elem;
        for (size_t k = 0; k < 16; ++k) {
            const uint8_t q = bp[2 + k];
            if (s + k < e) out[s + k] = (float)((int)(q & 0x0f) - 8) * scale;
            if (s + k + 16 < e) out[s + k + 16] = (float)((int)((q >> 4) & 0x0f) - 8) * scale;
        }
    }
}

void orc_q4_0_to_q4mat(const uint8_t* blocks, size_t n_elem, uint8_t* packed, float* scales) {
    const size_t nb = div_ceil(n_elem, 32);
    memset(packed, 0, div_ceil(n_elem, 2));
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* bp = blocks + b * 18;
        scales[b] = orc_f16_to_f32(rd16(bp));
        const size_t s = b * 32, e = s + 32 < n_elem ? s + 32 : n_elem;
        for (size_t k = 0; k < 16; ++k) {
            const uint8_t q = bp[2 + k];
            const size_t e0 = s + k, e1 = s + k + 16;
            const uint8_t v0 = (uint8_t)(((q & 0x0f) - 8) & 0x0f);
            const uint8_t v1 = (uint8_t)((((q >> 4) & 0x0f) - 8) & 0x0f);
            if (e0 < e) {
                if (e0 % 2 == 0)
                    packed[e0 / 2] = (uint8_t)((packed[e0 / 2] & 0xf0) | v0);
                else
                    packed[e0 / 2] = (uint8_t)((packed[e0 / 2] & 0x0f) | (v0 << 4));
            }
            if (e1 < e) {
                if (e1 % 2 == 0)
                    packed[e1 / 2] = (uint8_t)((packed[e1 / 2] & 0xf0) | v1);
                else
                    packed[e1 / 2] = (uint8_t)((packed[e1 / 2] & 0x0f) | (v1 << 4));
            }
        }
    }
}

void orc_q4_0_encode_block(const float* vals, float scale, uint8_t* out18) {
    const uint16_t s16 = orc_f32_to_f16(scale);
    out18[0] = (uint8_t)(s16 & 0xff);
    out18[1] = (uint8_t)(s16 >> 8);
    for (size_t k = 0; k < 16; ++k) {
        int q0 = (int)lroundf(vals[k] / scale) + 8;
        int q1 = (int)lroundf(vals[k + 16] / scale) + 8;
        q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
        q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
        out18[2 + k] = (uint8_t)(q0 | (q1 << 4));
    }
}

void orc_q4_0_quantize(const float* w, size_t n_elem, uint8_t* out) {
    /* Per 32 values: scale = absmax/7 (1 when zero), stored as (truncated)
     * f16; nibbles through the test encoder with the stored scale. */
    const size_t nb = n_elem / 32;
    for (size_t b = 0; b < nb; ++b) {
        const float* v = w + 32 * b;
        float amax = 0.0f;
        for (size_t i = 0; i < 32; ++i) amax = std_max(amax, fabsf(v[i]));
        const float scale = amax > 0.0f ? amax / 7.0f : 1.0f;
        orc_q4_0_encode_block(v, orc_f16_to_f32(orc_f32_to_f16(scale)), out + 18 * b);
    }
}

void orc_q6k_decode_f32(const uint8_t* blocks, size_t n_elem, float* out) {
    const size_t nb = div_ceil(n_elem, 256);
    memset(out, 0, n_elem * sizeof(float));
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* ql_all = blocks + b * 210;
        const uint8_t* qh_all = ql_all + 128;
        const int8_t* sc_all = (const int8_t*)(ql_all + 192);
        const float d = orc_f16_to_f32(rd16(ql_all + 208));
        const size_t base = b * 256, end = base + 256 < n_elem ? base + 256 : n_elem;
        for (size_t j = 0; j < 2; ++j) {
            const uint8_t* ql = ql_all + j * 64;
            const uint8_t* qh = qh_all + j * 32;
            const int8_t* sc = sc_all + j * 8;
            const size_t yb = base + j * 128;
            for (size_t l = 0; l < 32; ++l) {
                const size_t is = l / 16;
                const int q1 = (int)((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                const float s0 = d * (float)sc[is], s1 = d * (float)sc[is + 2];
                const float s2 = d * (float)sc[is + 4], s3 = d * (float)sc[is + 6];
                if (yb + l < end) out[yb + l] = s0 * (float)q1;
                if (yb + l + 32 < end) out[yb + l + 32] = s1 * (float)q2;
                if (yb + l + 64 < end) out[yb + l + 64] = s2 * (float)q3;
                if (yb + l + 96 < end) out[yb + l + 96] = s3 * (float)q4;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* argmax: src/transformer5.cpp:382-391                                     */
/* ------------------------------------------------------------------------ */

int64_t orc_argmax_first(const float* v, size_t n) {
    size_t best = 0;
    float best_v = -INFINITY;
    for (size_t c = 0; c < n; ++c) {
        if (v[c] > best_v) {
            best_v = v[c];
            best = c;
        }
    }
    return (int64_t)best;
}

/* ------------------------------------------------------------------------ */
/* Layer operations either side of a decode GEMV                            */
/* ------------------------------------------------------------------------ */

/* TensorNode::rms_norm / rms_norm_gemma3 on one row (src/tensor_node.cpp:
 * 320-344, 383-389): mean_sq summed in sequence in f32, times 1/d;
 * rms_inv = 1 / sqrt(mean_sq + eps); x_hat = x * rms_inv; out = x_hat * g,
 * g = gamma or 1 + gamma. */
void orc_rmsnorm(const float* x, const float* gamma, size_t d, float eps, int gemma3, float* out) {
    const float inv_d = 1.0f / (float)d;
    float mean_sq = 0.0f;
    for (size_t c = 0; c < d; ++c) mean_sq += x[c] * x[c];
    mean_sq *= inv_d;
    const float rms_inv = 1.0f / sqrtf(mean_sq + eps);
    for (size_t c = 0; c < d; ++c) {
        const float g = gemma3 ? 1.0f + gamma[c] : gamma[c];
        out[c] = (x[c] * rms_inv) * g;
    }
}

/* LlamaMlp::forward's activation (src/transformer5.cpp:186-190): silu(gate)
 * as TensorNode::silu computes it (src/tensor_node.cpp:391-402: the sigmoid
 * 1 / (1 + exp(-x)) first, then x * sigmoid), times up. */
void orc_swiglu(const float* gate, const float* up, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) {
        const float sig = 1.0f / (1.0f + expf(-gate[i]));
        out[i] = (gate[i] * sig) * up[i];
    }
}

/* Config5::inv_freq (src/transformer5.cpp:36-52): f = 1 / pow(theta,
 * 2i / head_dim) in f32, divided by divisors[i] where one is given (> 0). */
void orc_llama_inv_freq(float theta, size_t head_dim, const float* divisors, size_t n_div, float* out) {
    const size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        const float exponent = 2.0f * (float)i / (float)head_dim;
        float f = 1.0f / powf(theta, exponent);
        if (i < n_div && divisors[i] > 0.0f) f /= divisors[i];
        out[i] = f;
    }
}

/* llama_rope on one row, RopePairing::Interleaved (src/transformer5.cpp:
 * 95-125): for each pair i, a = pos * inv_freq[i], cos and sin of a, then
 * per head out[2i] = x0 cos - x1 sin, out[2i+1] = x0 sin + x1 cos. */
void orc_llama_rope_interleaved(const float* x, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq,
                                float* out) {
    const size_t half = head_dim / 2;
    memcpy(out, x, n_heads * head_dim * sizeof(float));
    for (size_t i = 0; i < half; ++i) {
        const float angle = (float)pos * inv_freq[i];
        const float c = cosf(angle), s = sinf(angle);
        for (size_t h = 0; h < n_heads; ++h) {
            const size_t c0 = h * head_dim + 2 * i, c1 = c0 + 1;
            const float x0 = x[c0], x1 = x[c1];
            out[c0] = x0 * c - x1 * s;
            out[c1] = x0 * s + x1 * c;
        }
    }
}

/* llama_rope on one row, RopePairing::HalfSplit (src/transformer5.cpp:
 * 95-125, the pairing of HuggingFace's weights): pair (i, i + head_dim/2)
 * of each head, a = pos * inv_freq[i], out_i = x0 cos - x1 sin,
 * out_{i+half} = x0 sin + x1 cos. */
void orc_llama_rope_half(const float* x, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq,
                         float* out) {
    const size_t half = head_dim / 2;
    memcpy(out, x, n_heads * head_dim * sizeof(float));
    for (size_t i = 0; i < half; ++i) {
        const float angle = (float)pos * inv_freq[i];
        const float c = cosf(angle), s = sinf(angle);
        for (size_t h = 0; h < n_heads; ++h) {
            const size_t c0 = h * head_dim + i, c1 = c0 + half;
            const float x0 = x[c0], x1 = x[c1];
            out[c0] = x0 * c - x1 * s;
            out[c1] = x0 * s + x1 * c;
        }
    }
}

/* gqa_attention_cached, decode path (src/transformer4.cpp:379-432): one
 * query row; for each query head, scores[c] = dot(q_h, k_h[c]) * scale over
 * c in [k_start, k_end) (sequential dot), max, exp(s - max) summed in order,
 * divided by the sum when positive, then out_h = sum_c p_c v_h[c] in order. */
void orc_gqa_attention_decode(const float* q, const float* k_cache, const float* v_cache, size_t k_start,
                              size_t k_end, size_t n_q_heads, size_t n_kv_heads, size_t d_head, float scale,
                              float* out) {
    const size_t t_kv = k_end - k_start, kv_stride = n_kv_heads * d_head, group = n_q_heads / n_kv_heads;
    float* scores = (float*)malloc((t_kv ? t_kv : 1) * sizeof(float));
    memset(out, 0, n_q_heads * d_head * sizeof(float));
    for (size_t qh = 0; qh < n_q_heads; ++qh) {
        const size_t kvh = qh / group, q_off = qh * d_head, kv_off = kvh * d_head, out_off = qh * d_head;
        for (size_t ci = 0; ci < t_kv; ++ci) {
            const size_t k_base = (k_start + ci) * kv_stride + kv_off;
            float dot = 0.0f;
            for (size_t di = 0; di < d_head; ++di) dot += q[q_off + di] * k_cache[k_base + di];
            scores[ci] = dot * scale;
        }
        float max_s = -INFINITY;
        for (size_t ci = 0; ci < t_kv; ++ci) max_s = max_s < scores[ci] ? scores[ci] : max_s;
        float sum_exp = 0.0f;
        for (size_t ci = 0; ci < t_kv; ++ci) {
            scores[ci] = expf(scores[ci] - max_s);
            sum_exp += scores[ci];
        }
        if (sum_exp > 0.0f)
            for (size_t ci = 0; ci < t_kv; ++ci) scores[ci] /= sum_exp;
        for (size_t ci = 0; ci < t_kv; ++ci) {
            const size_t v_base = (k_start + ci) * kv_stride + kv_off;
            for (size_t di = 0; di < d_head; ++di) out[out_off + di] += scores[ci] * v_cache[v_base + di];
        }
    }
    free(scores);
}

/* ------------------------------------------------------------------------ */
/* InitRng: include/rt/init_rng.hpp:14-47                                   */
/* ------------------------------------------------------------------------ */

static inline float rng_next_f32(uint64_t* st) {
    *st = *st * 6364136223846793005ull + 1442695040888963407ull;
    const uint32_t bits = (uint32_t)(*st >> 32);
    return (float)bits / (float)UINT32_MAX;
}

void orc_initrng_uniform(uint64_t seed, size_t n, float* out) {
    uint64_t st = seed + 1;
    for (size_t i = 0; i < n; ++i) out[i] = rng_next_f32(&st);
}

void orc_initrng_normal(uint64_t seed, size_t n, float std_dev, float* out) {
    uint64_t st = seed + 1;
    const float pi = 3.14159265358979323846f;
    for (size_t i = 0; i < n; ++i) {
        const float u1 = std_max(rng_next_f32(&st), 1e-7f);
        const float u2 = rng_next_f32(&st);
        const float r = sqrtf(-2.0f * logf(u1));
        const float theta = 2.0f * pi * u2;
        out[i] = r * cosf(theta) * std_dev;
    }
}

/* ---- Gemma 3 decode operations (the Metal engine, src/shaders/decode_gemma3.msl,
 * as src/metal_decode.mm:436-482 sequences them) -------------------------- */

/* rms_norm_per_head (decode_gemma3.msl:63-97): per head of head_dim values,
 * rms_inv = 1 / sqrt(sum(x^2) / head_dim + eps), out = x * rms_inv * (1 + gamma),
 * gamma [head_dim] shared by every head. */
void orc_rmsnorm_per_head(const float* x, const float* gamma, size_t n_heads, size_t head_dim, float eps,
                          float* out) {
    for (size_t h = 0; h < n_heads; ++h) {
        const float* xh = x + h * head_dim;
        float sq = 0.0f;
        for (size_t i = 0; i < head_dim; ++i) sq += xh[i] * xh[i];
        const float rms_inv = 1.0f / sqrtf(sq / (float)head_dim + eps);
        for (size_t i = 0; i < head_dim; ++i) out[h * head_dim + i] = xh[i] * rms_inv * (1.0f + gamma[i]);
    }
}

/* rope_neox (decode_gemma3.msl:99-126): pair (i, i + head_dim/2),
 * angle = (pos * freq_scale) / pow(theta, 2 i / head_dim), all in f32;
 * out_i = x0 cos - x1 sin, out_{i+half} = x0 sin + x1 cos. */
void orc_rope_neox(const float* x, size_t n_heads, size_t head_dim, float theta, float freq_scale, size_t pos,
                   float* out) {
    const size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        const float angle = ((float)pos * freq_scale) / powf(theta, 2.0f * (float)i / (float)head_dim);
        const float c = cosf(angle), s = sinf(angle);
        for (size_t h = 0; h < n_heads; ++h) {
            const size_t c0 = h * head_dim + i, c1 = c0 + half;
            const float x0 = x[c0], x1 = x[c1];
            out[c0] = x0 * c - x1 * s;
            out[c1] = x0 * s + x1 * c;
        }
    }
}

/* gelu_tanh_kernel (decode_gemma3.msl:128-145): the tanh approximation with
 * the argument of tanh clamped to [-10, 10]. */
void orc_gelu_tanh(const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) {
        const float v = x[i];
        const float v3 = v * v * v;
        float inner = 0.7978845608f * (v + 0.044715f * v3);
        inner = inner < -10.0f ? -10.0f : (inner > 10.0f ? 10.0f : inner);
        out[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* half(x) of the Metal KV-cache append (decode_gemma3.msl:174-187): IEEE
 * round to nearest even, overflow to infinity, subnormal halves kept.
 * (Not the truncating f32_to_f16 of bf16.hpp, which the Q4_K quantizer uses.) */
uint16_t orc_f32_to_f16_rne(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t absu = u & 0x7fffffffu;
    if (absu > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((absu >> 13) & 0x3ffu));  /* NaN */
    if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* rounds to >= 65520: inf */
    if (absu < 0x38800000u) {  /* below the smallest normal half: subnormal (or zero) */
        if (absu < 0x33000000u) return (uint16_t)sign;  /* below half of the smallest subnormal */
        const uint32_t mant = (absu & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - (absu >> 23);  /* so that the result is in units of 2^-24 */
        const uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
        const uint32_t r = q + ((rem > halfway || (rem == halfway && (q & 1u))) ? 1u : 0u);
        return (uint16_t)(sign | r);
    }
    const uint32_t e = (absu >> 23) - 112u;  /* rebias 127 -> 15 */
    const uint32_t m = absu & 0x7fffffu;
    uint32_t r = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

void orc_f32_to_f16_rne_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16_rne(src[i]);
}

/* FLUX attention (flux.cpp:287-321), per head h and output row i: the f32
 * dot products accumulated in key order times scale = 1/sqrt(head_dim)
 * (flux.cpp:290), the running maximum, exp(s - max) summed in key order,
 * inv = 1/denom, then out += (s_j * inv) * v_j in key order (out starts at
 * zero, flux.cpp:291). */
void orc_flux_attention(const float* q, const float* k, const float* v, size_t t, size_t n_heads,
                        size_t head_dim, const int64_t* rows, size_t n_rows, float* out) {
    const size_t width = n_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* scores = (float*)malloc((t ? t : 1) * sizeof(float));
    if (!scores) return;
    memset(out, 0, n_rows * width * sizeof(float));
    for (size_t h = 0; h < n_heads; ++h) {
        const size_t off = h * head_dim;
        for (size_t r = 0; r < n_rows; ++r) {
            const size_t i = rows ? (size_t)rows[r] : r;
            const float* qi = q + i * width + off;
            float max_score = -INFINITY;
            for (size_t j = 0; j < t; ++j) {
                const float* kj = k + j * width + off;
                float acc = 0.0f;
                for (size_t c = 0; c < head_dim; ++c) acc += qi[c] * kj[c];
                scores[j] = acc * scale;
                if (scores[j] > max_score) max_score = scores[j];
            }
            float denom = 0.0f;
            for (size_t j = 0; j < t; ++j) {
                scores[j] = expf(scores[j] - max_score);
                denom += scores[j];
            }
            const float inv = 1.0f / denom;
            float* dst = out + r * width + off;
            for (size_t j = 0; j < t; ++j) {
                const float weight = scores[j] * inv;
                const float* vj = v + j * width + off;
                for (size_t c = 0; c < head_dim; ++c) dst[c] += weight * vj[c];
            }
        }
    }
    free(scores);
}
