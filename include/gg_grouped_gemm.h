/*
 * C ABI of the MI355X (gfx950) persistent grouped GEMM.
 *
 * Op (the reference's forward MoE grouped GEMM, common/backend.hpp:32-38):
 *   x   [sum(group_m), k]  row-major   tokens of all groups, back to back
 *   w   [group_num, n, k]  row-major   one weight matrix per group
 *   out [sum(group_m), n]  row-major
 *   out[rows of group g] = x[rows of group g] @ w[g]^T
 * bf16 or fp16 in and out, fp32 accumulation, round-to-nearest-even on output.
 *
 * Plain pointers and sizes only: device pointers are addresses from hipMalloc (or any
 * allocator of device memory), `stream` is a hipStream_t passed as void* (NULL = the
 * default stream). Every entry point returns a gg_status; none exits the process.
 *
 * Life cycle, matching tunemax::Backend (common/backend.hpp:63-79):
 *   gg_prepare  -> Backend::prepare   (untimed: validate, build the device group table)
 *   gg_run      -> Backend::run       (timed: enqueue exactly one grouped GEMM, no sync)
 *   gg_release  -> Backend::release   (free what gg_prepare allocated)
 */
#ifndef GG_GROUPED_GEMM_H
#define GG_GROUPED_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of x, w and out. Same values as tunemax::DType (common/backend.hpp:27). */
typedef enum gg_dtype { GG_DTYPE_BF16 = 0, GG_DTYPE_FP16 = 1 } gg_dtype;

typedef enum gg_status {
    GG_OK = 0,
    /* The problem is valid but this kernel cannot run it; the message (gg_last_error) is the
     * reason, reported as "N/A" like a non-empty Backend::prepare result
     * (common/backend.hpp:63-66, bench/bench_main.cpp:469-472). */
    GG_ERR_UNSUPPORTED = 1,
    /* Bad arguments: null pointers, negative sizes, unknown dtype, null plan. */
    GG_ERR_INVALID = 2,
    /* A HIP runtime call failed (the reference's TUNEMAX_HIP_CHECK, common/backend.hpp:15-23,
     * prints and exits; this library returns the code and keeps the message). */
    GG_ERR_HIP = 3
} gg_status;

/* Opaque per-problem plan: device group table, launch shape, pointers. */
typedef struct gg_plan gg_plan;

/*
 * Validate the problem and build its plan. Replaces CkTileBackend::prepare_typed + finish
 * (ck_kernel/ck_grouped_gemm.cpp:153-218): per-group row offsets and tile ranges, one
 * hipMalloc + H2D copy of the argument table on `stream`, then a stream sync.
 *   group_m: host array of group_num row counts (>= 0; zero-row groups are skipped).
 *   x, w, out: device buffers laid out as above; they must stay valid while the plan is used.
 * Requirements (else GG_ERR_UNSUPPORTED): n % 8 == 0 and k % 8 == 0 (16-byte rows for the
 * 128-bit loads and stores), 16-byte aligned x, w and out.
 * k % 64 != 0 is supported (the reference rejects it, ck_grouped_gemm.cpp:192-193).
 * On success *plan_out owns device memory until gg_release.
 */
int gg_prepare(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
               const void *x, const void *w, void *out, void *stream, gg_plan **plan_out);

/*
 * Enqueue the grouped GEMM of `plan` on `stream`: one kernel launch, no host sync, no
 * allocation. Replaces CkTileBackend::run / CkGroupedGemm::launch
 * (ck_kernel/ck_grouped_gemm.cpp:140, 114-121). Problems with no output rows are a no-op;
 * k == 0 writes zeros.
 */
int gg_run(const gg_plan *plan, void *stream);

/* Free the plan and its device table. Replaces CkTileBackend::release
 * (ck_kernel/ck_grouped_gemm.cpp:142-146). NULL is accepted. */
void gg_release(gg_plan *plan);

/* Free-form note on the chosen kernel and launch (Backend::detail, common/backend.hpp:79).
 * The string lives as long as the plan. */
const char *gg_plan_detail(const gg_plan *plan);

/* Workgroups the plan launches and output tiles it covers (for tests and roofline math). */
int gg_plan_grid(const gg_plan *plan);
int gg_plan_tiles(const gg_plan *plan);

/* Message of the last failed call on the calling thread ("" if none). */
const char *gg_last_error(void);

/*
 * Seeded N(0,1) fill of `count` elements of `dtype` at device pointer p, deterministic in
 * (seed, index). The benchmark input generator of bench/bench_main.cpp:160-176, 451-456
 * (splitmix64 + Box-Muller; seeds 1 for x, 2 for w). Harness helper, not part of the op.
 */
int gg_fill_randn(int dtype, void *p, size_t count, uint64_t seed, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GG_GROUPED_GEMM_H */
