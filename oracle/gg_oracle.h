/*
 * CPU oracle for the grouped GEMM — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of what the reference computes and checks on this path. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as
 * the checker or the timed CPU baseline; the product (libgg_mi355x.so) never calls it.
 *
 * What each function follows (paths in the reference checkout):
 *   gg_oracle_grouped_gemm  common/backend.hpp:32-38 (op), bench/bench_main.cpp:185-206
 *                           (fp32 dot of x[row,:] and w[g][col,:]); ck_grouped_gemm.cpp:166-188
 *                           (group row offsets, w[g] at g*N*K)
 *   gg_oracle_sampled       bench/bench_main.cpp:185-206 (one fp32 dot per sample)
 *   gg_oracle_grouped_dgrad / gg_oracle_grouped_wgrad
 *                           the backward GEMMs of the same op, with the shapes of the vendored
 *                           Primus-Turbo grouped GEMM's check() (third_party/primus_turbo/kernels/
 *                           hipblaslt_grouped_gemm.cu:80-97: grad_c * b = grad_a, a^T * grad_c =
 *                           grad_b) and its zero output for an empty group's weight gradient
 *                           (:206-214); fp32 sums like gg_oracle_grouped_gemm
 *   gg_oracle_fp8_to_f32 / gg_oracle_grouped_gemm_fp8
 *                           the fp8 grouped GEMM with tensor-wise scales of the vendored
 *                           Primus-Turbo (third_party/primus_turbo/include/primus_turbo/
 *                           grouped_gemm.h:72-74, 120-123: aq_ptr / bq_ptr); fp8 formats are the
 *                           OCP e4m3 (bias 7, no infinities, 0x7f/0xff NaN) and e5m2 (bias 15)
 *   gg_oracle_grouped_dgrad_fp8 / gg_oracle_grouped_wgrad_fp8
 *                           its fp8 backward (grouped_gemm.h:123-130: ck_grouped_gemm_fp8 with a
 *                           transposed operand, ck_grouped_gemm_fp8_variable_k), per-operand
 *                           formats (the gradient may be e5m2 while w or x is e4m3)
 *   gg_oracle_make_samples  bench/bench_main.cpp:210-227 (4 corners + 256 random per group,
 *                           one std::mt19937_64(1234) engine for all groups)
 *   gg_oracle_check         bench/bench_main.cpp:235-271 (|got-ref| <= atol + rtol*|ref|, NaN is a
 *                           mismatch and makes max_abs infinite)
 *   gg_oracle_fill_randn    bench/bench_main.cpp:160-176 (splitmix64 + Box-Muller)
 *   gg_mt19937_64_*         the C++ standard's std::mt19937_64 ([rand.predef]), which the
 *                           reference's sampler uses
 *
 * Pinning (tests/test_oracle.py): fp8 decode against torch's float8_e4m3fn / float8_e5m2 on
 * all 256 patterns; mt19937_64 against the standard's known answer and against
 * libstdc++'s engine (tests/golden/); 16-bit decode/encode against numpy/torch; the GEMM
 * against numpy float64 matmul per group and against exact integer known answers; the
 * sampler and the check by their specification's invariants and hand-built cases.
 * Parity unpinned: gg_oracle_fill_randn's exact bits (the reference's device logf/cospif are
 * not reproducible on the host); it is pinned only statistically and by its agreement with
 * the device generator to within one 16-bit ulp.
 */
#ifndef GG_ORACLE_H
#define GG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype: 0 = bf16, 1 = fp16 (same values as gg_dtype). */

float    gg_oracle_bf16_to_f32(uint16_t h);
float    gg_oracle_f16_to_f32(uint16_t h);
uint16_t gg_oracle_f32_to_bf16(float f); /* round to nearest even, NaN stays NaN */
uint16_t gg_oracle_f32_to_f16(float f);  /* round to nearest even, overflow -> inf */
void     gg_oracle_decode(int dtype, const uint16_t *src, float *dst, size_t count);
void     gg_oracle_encode(int dtype, const float *src, uint16_t *dst, size_t count);

/* out[row, col] (fp32) = sum_k x[row, k] * w[g, col, k] for every row of every group.
 * x: [sum(group_m), k], w: [group_num, n, k], out: [sum(group_m), n]. OpenMP over rows. */
void gg_oracle_grouped_gemm(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                            const uint16_t *x, const uint16_t *w, float *out);

/* Input gradient: out[row, c] (fp32) = sum_j grad_out[row, j] * w[g, j, c] for every row of
 * every group. grad_out: [sum(group_m), n], w: [group_num, n, k], out: [sum(group_m), k]. */
void gg_oracle_grouped_dgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                             const uint16_t *grad_out, const uint16_t *w, float *out);

/* Weight gradient: out[g, i, c] (fp32) = sum over the rows r of group g of grad_out[r, i] *
 * x[r, c]; zero for an empty group. grad_out: [sum(group_m), n], x: [sum(group_m), k],
 * out: [group_num, n, k]. */
void gg_oracle_grouped_wgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                             const uint16_t *grad_out, const uint16_t *x, float *out);

/* fp8 (fmt 0: e4m3, 1: e5m2) -> fp32, exact. */
float gg_oracle_fp8_to_f32(int fmt, uint8_t b);

/* out[row, col] (fp32) = (sum_k x[row, k] * w[g, col, k]) * x_scale * w_scale[g], fp8 inputs. */
void gg_oracle_grouped_gemm_fp8(int fmt, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                                const uint8_t *x, const uint8_t *w, float x_scale, const float *w_scale,
                                float *out);

/* fp8 input gradient: out[row, c] (fp32) = (sum_j grad_out[row, j] * w[g, j, c]) * a_scale *
 * b_scale[g]; grad_out [sum(group_m), n] in format a_fmt, w [group_num, n, k] in b_fmt. */
void gg_oracle_grouped_dgrad_fp8(int a_fmt, int b_fmt, int group_num, int64_t n, int64_t k,
                                 const int64_t *group_m, const uint8_t *grad_out, const uint8_t *w,
                                 float a_scale, const float *b_scale, float *out);

/* fp8 weight gradient: out[g, i, c] (fp32) = (sum over the rows r of group g of grad_out[r, i] *
 * x[r, c]) * a_scale * b_scale[g], zero for an empty group; grad_out [sum(group_m), n] in a_fmt,
 * x [sum(group_m), k] in b_fmt, out [group_num, n, k]. */
void gg_oracle_grouped_wgrad_fp8(int a_fmt, int b_fmt, int group_num, int64_t n, int64_t k,
                                 const int64_t *group_m, const uint8_t *grad_out, const uint8_t *x,
                                 float a_scale, const float *b_scale, float *out);

/* Same dot products for rows [row_begin, row_end) of one group only (out: [rows, n]).
 * The bounded CPU baseline sample. */
void gg_oracle_group_rows(int dtype, int64_t n, int64_t k, const uint16_t *x_rows,
                          const uint16_t *w_group, int64_t rows, float *out);

/* One fp32 dot per sample: samples[3*i .. 3*i+2] = (row, col, group). */
void gg_oracle_sampled(int dtype, int64_t n, int64_t k, const uint16_t *x, const uint16_t *w,
                       const int64_t *samples, int64_t count, float *ref);

/* Sample positions of the reference driver. Writes (row, col, group) triples to `out` (may be
 * NULL to only count) and returns the number of samples. */
int64_t gg_oracle_make_samples(int group_num, int64_t n, const int64_t *group_m, int per_group,
                               int64_t *out);

/* Mismatch count under |got - ref| <= atol + rtol * |ref|; *max_abs gets the largest error
 * (infinity if any error is NaN). */
int64_t gg_oracle_check(const float *got, const float *ref, int64_t count, double atol, double rtol,
                        double *max_abs);

/* Seeded N(0,1) generator of the reference driver, restated on the host. */
void gg_oracle_fill_randn(int dtype, uint16_t *p, size_t count, uint64_t seed);
/* The generator's splitmix64 stage alone: mix(z + 0x9E3779B97F4A7C15), i.e. the next output of a
 * splitmix64 whose state is z (bench/bench_main.cpp:160-165). */
uint64_t gg_oracle_splitmix64(uint64_t z);

/* std::mt19937_64: `count` outputs of an engine seeded with `seed`. */
void gg_mt19937_64_seq(uint64_t seed, uint64_t *out, size_t count);
/* The z-th output (1-based) of an engine seeded with `seed`. */
uint64_t gg_mt19937_64_nth(uint64_t seed, uint64_t z);

/* Threads the OpenMP loops use. */
int gg_oracle_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* GG_ORACLE_H */
