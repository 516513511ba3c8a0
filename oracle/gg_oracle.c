/*
 * CPU oracle for the grouped GEMM — TEST INFRASTRUCTURE ONLY (see gg_oracle.h for what each
 * function restates, where in the reference, and how it is pinned).
 */
#include "gg_oracle.h"

#include <math.h>
#include <omp.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------
 * 16-bit floating point formats
 * ------------------------------------------------------------------------------------- */
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* bf16 is the upper half of an IEEE binary32. */
float gg_oracle_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* IEEE binary16: 1 sign, 5 exponent (bias 15), 10 fraction bits. */
float gg_oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp  = (h >> 10) & 0x1f;
    const uint32_t frac = h & 0x3ff;
    if (exp == 0x1f) /* inf / NaN */
        return bits_f32(sign | 0x7f800000u | (frac << 13));
    if (exp != 0) /* normal */
        return bits_f32(sign | ((exp + 112) << 23) | (frac << 13));
    /* zero or subnormal: frac * 2^-24 */
    const float v = (float)frac * 5.9604644775390625e-08f;
    return sign ? -v : v;
}

uint16_t gg_oracle_f32_to_bf16(float f) {
    const uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) /* NaN: keep it a (quiet) NaN */
        return (uint16_t)((u >> 16) | 0x40);
    /* round to nearest, ties to even, on the 16 dropped bits */
    const uint32_t rounded = u + 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

uint16_t gg_oracle_f32_to_f16(float f) {
    const uint32_t u    = f32_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a    = u & 0x7fffffffu;
    if (a > 0x7f800000u) /* NaN */
        return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) /* rounds to >= 65520: overflow to infinity */
        return (uint16_t)(sign | 0x7c00u);
    if (a >= 0x38800000u) { /* normal half: exponent >= -14 */
        const uint32_t e = (a >> 23) - 112;      /* half exponent field */
        uint32_t       m = a & 0x7fffffu;        /* 23-bit fraction */
        uint32_t       h = (e << 10) | (m >> 13);
        const uint32_t rest = m & 0x1fffu;       /* 13 dropped bits */
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u)))
            ++h; /* may carry into the exponent, which is still correct */
        return (uint16_t)(sign | h);
    }
    /* subnormal half (or zero): value / 2^-24, rounded to nearest even integer */
    const double q = (double)bits_f32(a) * 16777216.0; /* exact in double */
    double       r = floor(q);
    const double d = q - r;
    if (d > 0.5 || (d == 0.5 && fmod(r, 2.0) != 0.0))
        r += 1.0;
    return (uint16_t)(sign | (uint16_t)r); /* r <= 1024 reaches the smallest normal */
}

void gg_oracle_decode(int dtype, const uint16_t *src, float *dst, size_t count) {
#pragma omp parallel for schedule(static) if (count > 65536)
    for (size_t i = 0; i < count; ++i)
        dst[i] = dtype == 0 ? gg_oracle_bf16_to_f32(src[i]) : gg_oracle_f16_to_f32(src[i]);
}

void gg_oracle_encode(int dtype, const float *src, uint16_t *dst, size_t count) {
#pragma omp parallel for schedule(static) if (count > 65536)
    for (size_t i = 0; i < count; ++i)
        dst[i] = dtype == 0 ? gg_oracle_f32_to_bf16(src[i]) : gg_oracle_f32_to_f16(src[i]);
}

/* ---------------------------------------------------------------------------------------
 * fp32 grouped GEMM
 * ------------------------------------------------------------------------------------- */
typedef float v8f __attribute__((vector_size(32)));

static inline float hsum8(v8f v) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

/* Rows r0..r0+3 (clamped by `rows`) of xf against columns c0..c0+3 of wf, K-contiguous. */
static void dot_block(const float *xf, const float *wf, int64_t k, int64_t rows, int64_t cols,
                      int64_t r0, int64_t c0, float *out, int64_t ldo) {
    v8f    acc[4][4];
    const float *xr[4], *wr[4];
    memset(acc, 0, sizeof(acc));
    for (int i = 0; i < 4; ++i) {
        xr[i] = xf + (r0 + (r0 + i < rows ? i : 0)) * k;
        wr[i] = wf + (c0 + (c0 + i < cols ? i : 0)) * k;
    }
    int64_t kk = 0;
    for (; kk + 8 <= k; kk += 8) {
        v8f xv[4], wv[4];
        for (int i = 0; i < 4; ++i) {
            memcpy(&xv[i], xr[i] + kk, 32);
            memcpy(&wv[i], wr[i] + kk, 32);
        }
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j)
                acc[i][j] += xv[i] * wv[j];
    }
    for (int i = 0; i < 4 && r0 + i < rows; ++i)
        for (int j = 0; j < 4 && c0 + j < cols; ++j) {
            float s = hsum8(acc[i][j]);
            for (int64_t t = kk; t < k; ++t)
                s += xr[i][t] * wr[j][t];
            out[(r0 + i) * ldo + c0 + j] = s;
        }
}

/* rows x n block of one group from decoded operands; columns blocked for cache reuse. */
static void group_block(const float *xf, const float *wf, int64_t rows, int64_t n, int64_t k,
                        float *out) {
    const int64_t cb = 64; /* columns per cache block */
    const int64_t row_blocks = (rows + 3) / 4, col_blocks = (n + cb - 1) / cb;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t rb = 0; rb < row_blocks; ++rb)
        for (int64_t c = 0; c < col_blocks; ++c)
            for (int64_t c0 = c * cb; c0 < (c + 1) * cb && c0 < n; c0 += 4)
                dot_block(xf, wf, k, rows, n, rb * 4, c0, out, n);
}

#include <stdlib.h>

void gg_oracle_group_rows(int dtype, int64_t n, int64_t k, const uint16_t *x_rows,
                          const uint16_t *w_group, int64_t rows, float *out) {
    if (rows <= 0 || n <= 0)
        return;
    if (k == 0) {
        memset(out, 0, (size_t)(rows * n) * sizeof(float));
        return;
    }
    float *xf = (float *)malloc((size_t)(rows * k) * sizeof(float));
    float *wf = (float *)malloc((size_t)(n * k) * sizeof(float));
    gg_oracle_decode(dtype, x_rows, xf, (size_t)(rows * k));
    gg_oracle_decode(dtype, w_group, wf, (size_t)(n * k));
    group_block(xf, wf, rows, n, k, out);
    free(xf);
    free(wf);
}

void gg_oracle_grouped_gemm(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                            const uint16_t *x, const uint16_t *w, float *out) {
    int64_t row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t m = group_m[g];
        if (m > 0)
            gg_oracle_group_rows(dtype, n, k, x + row0 * k, w + (int64_t)g * n * k, m,
                                 out + row0 * n);
        row0 += m;
    }
}

float gg_oracle_fp8_to_f32(int fmt, uint8_t b) {
    const int   sign = b >> 7;
    const int   eb   = fmt == 0 ? 4 : 5, mb = fmt == 0 ? 3 : 2, bias = fmt == 0 ? 7 : 15;
    const int   e    = (b >> mb) & ((1 << eb) - 1), m = b & ((1 << mb) - 1);
    float       v;
    if (fmt == 0 && e == 15 && m == 7)
        v = NAN; /* e4m3: the only NaN, no infinities */
    else if (fmt == 1 && e == 31)
        v = m == 0 ? INFINITY : NAN;
    else if (e == 0)
        v = ldexpf((float)m, 1 - bias - mb); /* subnormal: m * 2^(1 - bias - mb) */
    else
        v = ldexpf((float)((1 << mb) + m), e - bias - mb);
    return sign ? -v : v;
}

void gg_oracle_grouped_gemm_fp8(int fmt, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                                const uint8_t *x, const uint8_t *w, float x_scale, const float *w_scale,
                                float *out) {
    float lut[256];
    for (int i = 0; i < 256; ++i)
        lut[i] = gg_oracle_fp8_to_f32(fmt, (uint8_t)i);
    int64_t row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t  m  = group_m[g];
        const uint8_t *wg = w + (int64_t)g * n * k;
        const float    sc = x_scale * w_scale[g];
#pragma omp parallel for schedule(static)
        for (int64_t r = row0; r < row0 + m; ++r) {
            const uint8_t *xr = x + r * k;
            for (int64_t c = 0; c < n; ++c) {
                const uint8_t *wr = wg + c * k;
                float          s  = 0.f;
                for (int64_t t = 0; t < k; ++t)
                    s += lut[xr[t]] * lut[wr[t]];
                out[r * n + c] = s * sc;
            }
        }
        row0 += m;
    }
}

static void fp8_lut(int fmt, float *lut) {
    for (int i = 0; i < 256; ++i)
        lut[i] = gg_oracle_fp8_to_f32(fmt, (uint8_t)i);
}

/* Follows gg_oracle_grouped_dgrad below with fp8 decode and the two scales. */
void gg_oracle_grouped_dgrad_fp8(int a_fmt, int b_fmt, int group_num, int64_t n, int64_t k,
                                 const int64_t *group_m, const uint8_t *grad_out, const uint8_t *w,
                                 float a_scale, const float *b_scale, float *out) {
    float la[256], lb[256];
    fp8_lut(a_fmt, la);
    fp8_lut(b_fmt, lb);
    int64_t row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t  m  = group_m[g];
        const uint8_t *wg = w + (int64_t)g * n * k;
        const float    sc = a_scale * b_scale[g];
#pragma omp parallel for schedule(static)
        for (int64_t r = row0; r < row0 + m; ++r) {
            float *o = out + r * k;
            for (int64_t c = 0; c < k; ++c)
                o[c] = 0.f;
            for (int64_t j = 0; j < n; ++j) {
                const float    a  = la[grad_out[r * n + j]];
                const uint8_t *wr = wg + j * k;
                for (int64_t c = 0; c < k; ++c)
                    o[c] += a * lb[wr[c]];
            }
            for (int64_t c = 0; c < k; ++c)
                o[c] *= sc;
        }
        row0 += m;
    }
}

/* Follows gg_oracle_grouped_wgrad below with fp8 decode and the two scales. */
void gg_oracle_grouped_wgrad_fp8(int a_fmt, int b_fmt, int group_num, int64_t n, int64_t k,
                                 const int64_t *group_m, const uint8_t *grad_out, const uint8_t *x,
                                 float a_scale, const float *b_scale, float *out) {
    float la[256], lb[256];
    fp8_lut(a_fmt, la);
    fp8_lut(b_fmt, lb);
    int64_t row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t m  = group_m[g];
        const float   sc = a_scale * b_scale[g];
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float *o = out + ((int64_t)g * n + i) * k;
            for (int64_t c = 0; c < k; ++c)
                o[c] = 0.f;
            for (int64_t r = row0; r < row0 + m; ++r) {
                const float    a  = la[grad_out[r * n + i]];
                const uint8_t *xr = x + r * k;
                for (int64_t c = 0; c < k; ++c)
                    o[c] += a * lb[xr[c]];
            }
            for (int64_t c = 0; c < k; ++c)
                o[c] *= sc;
        }
        row0 += m;
    }
}

static inline float dec(int dtype, uint16_t h) {
    return dtype == 0 ? gg_oracle_bf16_to_f32(h) : gg_oracle_f16_to_f32(h);
}

void gg_oracle_grouped_dgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                             const uint16_t *grad_out, const uint16_t *w, float *out) {
    int64_t row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t   m  = group_m[g];
        const uint16_t *wg = w + (int64_t)g * n * k;
#pragma omp parallel for schedule(static)
        for (int64_t r = row0; r < row0 + m; ++r) {
            float *o = out + r * k;
            for (int64_t c = 0; c < k; ++c)
                o[c] = 0.f;
            for (int64_t j = 0; j < n; ++j) {
                const float a = dec(dtype, grad_out[r * n + j]);
                const uint16_t *wr = wg + j * k;
                for (int64_t c = 0; c < k; ++c)
                    o[c] += a * dec(dtype, wr[c]);
            }
        }
        row0 += m;
    }
}

void gg_oracle_grouped_wgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                             const uint16_t *grad_out, const uint16_t *x, float *out) {
    int64_t row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t m = group_m[g];
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float *o = out + ((int64_t)g * n + i) * k;
            for (int64_t c = 0; c < k; ++c)
                o[c] = 0.f;
            for (int64_t r = row0; r < row0 + m; ++r) {
                const float a = dec(dtype, grad_out[r * n + i]);
                const uint16_t *xr = x + r * k;
                for (int64_t c = 0; c < k; ++c)
                    o[c] += a * dec(dtype, xr[c]);
            }
        }
        row0 += m;
    }
}

void gg_oracle_sampled(int dtype, int64_t n, int64_t k, const uint16_t *x, const uint16_t *w,
                       const int64_t *samples, int64_t count, float *ref) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        const uint16_t *xr = x + samples[3 * i] * k;
        const uint16_t *wr = w + (samples[3 * i + 2] * n + samples[3 * i + 1]) * k;
        float s = 0.f;
        for (int64_t t = 0; t < k; ++t) {
            const float a = dtype == 0 ? gg_oracle_bf16_to_f32(xr[t]) : gg_oracle_f16_to_f32(xr[t]);
            const float b = dtype == 0 ? gg_oracle_bf16_to_f32(wr[t]) : gg_oracle_f16_to_f32(wr[t]);
            s += a * b;
        }
        ref[i] = s;
    }
}

/* ---------------------------------------------------------------------------------------
 * std::mt19937_64 (C++ standard [rand.eng.mers] with the [rand.predef] parameters:
 * w=64 n=312 m=156 r=31 a=0xb5026f5aa96619e9 u=29 d=0x5555555555555555 s=17
 * b=0x71d67fffeda60000 t=37 c=0xfff7eee000000000 l=43 f=6364136223846793005)
 * ------------------------------------------------------------------------------------- */
#define MT_N 312
#define MT_M 156
typedef struct {
    uint64_t x[MT_N];
    int      i;
} mt64;

static void mt64_seed(mt64 *e, uint64_t seed) {
    e->x[0] = seed;
    for (int i = 1; i < MT_N; ++i)
        e->x[i] = 6364136223846793005ull * (e->x[i - 1] ^ (e->x[i - 1] >> 62)) + (uint64_t)i;
    e->i = 0;
}

static uint64_t mt64_next(mt64 *e) {
    const uint64_t upper = 0xffffffff80000000ull, lower = 0x7fffffffull; /* r = 31 */
    const int      i     = e->i;
    const uint64_t y     = (e->x[i] & upper) | (e->x[(i + 1) % MT_N] & lower);
    uint64_t       v     = e->x[(i + MT_M) % MT_N] ^ (y >> 1) ^ ((y & 1u) ? 0xb5026f5aa96619e9ull : 0);
    e->x[i]              = v;
    e->i                 = (i + 1) % MT_N;
    v ^= (v >> 29) & 0x5555555555555555ull;
    v ^= (v << 17) & 0x71d67fffeda60000ull;
    v ^= (v << 37) & 0xfff7eee000000000ull;
    v ^= v >> 43;
    return v;
}

void gg_mt19937_64_seq(uint64_t seed, uint64_t *out, size_t count) {
    mt64 e;
    mt64_seed(&e, seed);
    for (size_t i = 0; i < count; ++i)
        out[i] = mt64_next(&e);
}

uint64_t gg_mt19937_64_nth(uint64_t seed, uint64_t z) {
    mt64 e;
    mt64_seed(&e, seed);
    uint64_t v = 0;
    for (uint64_t i = 0; i < z; ++i)
        v = mt64_next(&e);
    return v;
}

/* ---------------------------------------------------------------------------------------
 * Sampler and check of the reference driver
 * ------------------------------------------------------------------------------------- */
int64_t gg_oracle_make_samples(int group_num, int64_t n, const int64_t *group_m, int per_group,
                               int64_t *out) {
    mt64 e;
    mt64_seed(&e, 1234);
    int64_t cnt = 0, row0 = 0;
    for (int g = 0; g < group_num; ++g) {
        const int64_t m = group_m[g];
        if (m > 0) {
            const int64_t rows[2] = {row0, row0 + m - 1}, cols[2] = {0, n - 1};
            for (int a = 0; a < 2; ++a)
                for (int b = 0; b < 2; ++b) {
                    if (out) {
                        out[3 * cnt]     = rows[a];
                        out[3 * cnt + 1] = cols[b];
                        out[3 * cnt + 2] = g;
                    }
                    ++cnt;
                }
            for (int i = 0; i < per_group; ++i) {
                const uint64_t r = mt64_next(&e); /* row draw first, then column */
                const uint64_t c = mt64_next(&e);
                if (out) {
                    out[3 * cnt]     = row0 + (int64_t)(r % (uint64_t)m);
                    out[3 * cnt + 1] = (int64_t)(c % (uint64_t)n);
                    out[3 * cnt + 2] = g;
                }
                ++cnt;
            }
        }
        row0 += m;
    }
    return cnt;
}

int64_t gg_oracle_check(const float *got, const float *ref, int64_t count, double atol, double rtol,
                        double *max_abs) {
    int64_t bad = 0;
    double  mx  = 0.0;
    for (int64_t i = 0; i < count; ++i) {
        const double err = fabs((double)got[i] - (double)ref[i]);
        const double e   = isnan(err) ? INFINITY : err;
        if (e > mx)
            mx = e;
        if (!(err <= atol + rtol * fabs((double)ref[i])))
            ++bad;
    }
    if (max_abs)
        *max_abs = mx;
    return bad;
}

/* ---------------------------------------------------------------------------------------
 * Input generator of the reference driver: splitmix64 (Steele, Lea, Flood 2014; constants
 * as published by Vigna) of seed ^ (index * 0x2545F4914F6CDD1D), then Box-Muller.
 * ------------------------------------------------------------------------------------- */
static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t gg_oracle_splitmix64(uint64_t z) { return splitmix64(z); }

void gg_oracle_fill_randn(int dtype, uint16_t *p, size_t count, uint64_t seed) {
#pragma omp parallel for schedule(static) if (count > 65536)
    for (size_t i = 0; i < count; ++i) {
        const uint64_t r  = splitmix64(seed ^ ((uint64_t)i * 0x2545F4914F6CDD1Dull));
        const float    u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777217.0f);
        const float    u2 = (float)((r >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
        const float    v  = (float)(sqrt(-2.0 * log((double)u1)) * cos(2.0 * M_PI * (double)u2));
        p[i] = dtype == 0 ? gg_oracle_f32_to_bf16(v) : gg_oracle_f32_to_f16(v);
    }
}

int gg_oracle_threads(void) { return omp_get_max_threads(); }
