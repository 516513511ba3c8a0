/*
 * C ABI of the comparison backends (lib/libgg_compare.so), for drivers that are not C++ (bench.py
 * times them in the same process, on the same buffers, right after the MI355X kernel). Not part
 * of the product boundary (include/gg_grouped_gemm.h): these are the hipBLASLt baselines the
 * reference measures its kernel against (README.md:54-58), behind its Backend contract
 * (common/backend.hpp:63-79): prepare untimed, run enqueues one grouped GEMM without a sync.
 *
 * Status: 0 ok, 1 N/A (the backend cannot run this problem; ggc_message says why), 2 error (a
 * HIP or hipBLASLt call failed; ggc_message holds it). No call exits the process.
 */
#ifndef GG_COMPARE_H
#define GG_COMPARE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggc_backend ggc_backend;

/* name: "hipblaslt_loop" (4 streams), "hipblaslt_seq" (1 stream) or "hipblaslt_grouped". */
int ggc_create(const char *name, ggc_backend **out);
/* dtype 0 bf16, 1 fp16; group_m host sizes; group_lens_pinned the same values in pinned host
 * memory (read by the per-group loops on every run); x, w, out device buffers (RCR layout). */
int ggc_prepare(ggc_backend *b, int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                const int64_t *group_lens_pinned, const void *x, const void *w, void *out, void *stream);
int ggc_run(ggc_backend *b, void *stream);
void ggc_release(ggc_backend *b);
void ggc_destroy(ggc_backend *b);
const char *ggc_message(const ggc_backend *b);
const char *ggc_detail(const ggc_backend *b);
/* The hipBLASLt heuristic's first kernel for one group (out^T [n x m] = w^T x^T, depth k), by
 * name into buf, without a launch: 1 if it is a stream-K kernel, 0 if not, -1 on failure. */
/* 1 if kernel_name names a stream-K solution (Tensile token "_SK<n>_" with n > 0), else 0. */
int ggc_is_stream_k(const char *kernel_name);
int ggc_heuristic_kernel(int dtype, int64_t n, int64_t m, int64_t k, char *buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* GG_COMPARE_H */
