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

/* Element type of x, w and out. BF16 and FP16: same values as tunemax::DType
 * (common/backend.hpp:27). The fp8 types are inputs of the fp8 entry points only (out is bf16). */
typedef enum gg_dtype {
    GG_DTYPE_BF16     = 0,
    GG_DTYPE_FP16     = 1,
    GG_DTYPE_FP8_E4M3 = 2, /* OCP e4m3 (finite, max 448) */
    GG_DTYPE_FP8_E5M2 = 3  /* OCP e5m2 */
} gg_dtype;

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
 * (ck_kernel/ck_grouped_gemm.cpp:153-218): per-group row offsets and tile ranges, a hipMalloc
 * + H2D copy of the argument table on `stream` (and of the per-workgroup tile descriptors, and
 * the fp32 workspace of a split-K or tail-split plan), then a stream sync.
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
 * Enqueue the grouped GEMM of `plan` on `stream`: one kernel launch (two for a split-K or
 * tail-split plan: the GEMM, then the reduction of its partial sums), no host sync, no
 * allocation. Replaces CkTileBackend::run / CkGroupedGemm::launch
 * (ck_kernel/ck_grouped_gemm.cpp:140, 114-121). Problems with no output rows are a no-op;
 * k == 0 writes zeros.
 */
int gg_run(const gg_plan *plan, void *stream);

/*
 * Backward GEMMs of the same op, for the MoE layer's backward pass (the reference's driver
 * times the forward only, README.md:35-36; the vendored Primus-Turbo grouped GEMM has both with
 * these shapes, third_party/primus_turbo/kernels/hipblaslt_grouped_gemm.cu:80-97, 206-214, and
 * a variable-K CK entry point for the weight gradient,
 * third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:115-116).
 *
 * gg_prepare_dgrad: grad_x[rows of g] [M_g, k] = grad_out[rows of g] [M_g, n] @ w[g] [n, k]
 *   grad_out [sum(group_m), n], w [group_num, n, k] (the forward's w), grad_x [sum(group_m), k].
 * gg_prepare_wgrad: grad_w[g] [n, k] = grad_out[rows of g]^T [n, M_g] @ x[rows of g] [M_g, k],
 *   grad_out [sum(group_m), n], x [sum(group_m), k], grad_w [group_num, n, k]; zero for an empty
 *   group (the contraction length of each group is its row count).
 * Same conventions as gg_prepare (host group_m, status codes, gg_run / gg_release), and the
 * same N/A rules: n and k multiples of 8 and at most 2097152, 16-byte aligned buffers; further
 * N/A: one group's w (dgrad) or one group's rows of grad_out or x (wgrad) of 2 GiB or more.
 */
int gg_prepare_dgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                     const void *grad_out, const void *w, void *grad_x, void *stream, gg_plan **plan_out);
int gg_prepare_wgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                     const void *grad_out, const void *x, void *grad_w, void *stream, gg_plan **plan_out);

/*
 * fp8 forward with tensor-wise scales: out[rows of g] (bf16) = (x[rows of g] @ w[g]^T) *
 * x_scale[0] * w_scale[g], x and w fp8 (dtype GG_DTYPE_FP8_E4M3 or GG_DTYPE_FP8_E5M2, both the
 * same), fp32 accumulation; x_scale (1 float) and w_scale (group_num floats) are device memory,
 * read by every run. Replaces primus_turbo::ck_grouped_gemm_fp8 with its aq_ptr / bq_ptr scales
 * (third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:72-74, 120-123). Same plan
 * life cycle as gg_prepare; N/A unless k % 16 == 0 (16-byte input rows) and n % 8 == 0.
 */
int gg_prepare_fp8(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                   const void *x, const void *w, const float *x_scale, const float *w_scale, void *out,
                   void *stream, gg_plan **plan_out);

/*
 * fp8 backward, the shapes of gg_prepare_dgrad / gg_prepare_wgrad with fp8 inputs and a bf16
 * output scaled by grad_scale[0] * w_scale[g] (dgrad) or grad_scale[0] * x_scale[g] (wgrad):
 * device scales, one for grad_out, one per group for the other operand (repeat a tensor-wise
 * scale). Formats (grad_dtype x w_dtype / x_dtype): e4m3 x e4m3, e5m2 x e5m2, or the hybrid
 * recipe's e5m2 gradient x e4m3. Replaces primus_turbo::ck_grouped_gemm_fp8 with a transposed
 * operand and ck_grouped_gemm_fp8_variable_k
 * (third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:123-130, with the aq_ptr /
 * bq_ptr scales of :72-74). Same plan life cycle as gg_prepare; N/A unless n and k are multiples
 * of 16, plus the 2 GiB rules of gg_prepare_dgrad / gg_prepare_wgrad.
 */
int gg_prepare_dgrad_fp8(int grad_dtype, int w_dtype, int group_num, int64_t n, int64_t k,
                         const int64_t *group_m, const void *grad_out, const void *w, const float *grad_scale,
                         const float *w_scale, void *grad_x, void *stream, gg_plan **plan_out);
int gg_prepare_wgrad_fp8(int grad_dtype, int x_dtype, int group_num, int64_t n, int64_t k,
                         const int64_t *group_m, const void *grad_out, const void *x, const float *grad_scale,
                         const float *x_scale, void *grad_w, void *stream, gg_plan **plan_out);

/* Free the plan and its device table. Replaces CkTileBackend::release
 * (ck_kernel/ck_grouped_gemm.cpp:142-146). NULL is accepted. */
void gg_release(gg_plan *plan);

/* Free-form note on the chosen kernel and launch (Backend::detail, common/backend.hpp:79).
 * The string lives as long as the plan. */
const char *gg_plan_detail(const gg_plan *plan);

/* Workgroups the plan launches and output tiles it covers (for tests and roofline math). */
int gg_plan_grid(const gg_plan *plan);
int gg_plan_tiles(const gg_plan *plan);

/*
 * Device-resident group sizes (the output of MoE routing, never read on the host): like
 * gg_prepare, but the sizes stay in device memory and every gg_run re-reads them on its stream,
 * so one plan serves every routing of a layer. Replaces the group_lens_ptr / group_offs_ptr
 * contract of the reference's vendored Primus-Turbo grouped GEMM
 * (third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:35-36, 95-96; read per call in
 * kernels/hipblaslt_grouped_gemm.cu:174-216).
 *   group_lens: device int64[group_num], rows of each group.
 *   group_offs: device int64[group_num + 1], first row of each group, or NULL: the groups are
 *               back to back from row 0 (offsets = prefix sums of group_lens).
 *   total_m:    rows of x and out. A group with a negative length, or rows outside
 *               [0, total_m), gets no work (its rows are not written) and is reported by
 *               gg_plan_device_status.
 * With group_num <= 64 each gg_run is one launch (the grouped GEMM builds the group table
 * itself); with more groups it is two: a one-wave table build, then the grouped GEMM. k == 0
 * zeroes all total_m rows of out. Same shape requirements as gg_prepare.
 */
int gg_prepare_device_lens(int dtype, int group_num, int64_t total_m, int64_t n, int64_t k,
                           const int64_t *group_lens, const int64_t *group_offs, const void *x,
                           const void *w, void *out, void *stream, gg_plan **plan_out);

/* Passes of gg_prepare_device_lens_op. */
typedef enum gg_op {
    GG_OP_FORWARD = 0, /* out = x @ w[g]^T: a = x [total_m, k], b = w [group_num, n, k], out [total_m, n] */
    GG_OP_DGRAD   = 1, /* grad_x = grad_out @ w[g]: a = grad_out [total_m, n], b = w, out [total_m, k] */
    GG_OP_WGRAD   = 2  /* grad_w[g] = grad_out[g]^T @ x[g]: a = grad_out [total_m, n], b = x [total_m, k],
                          out [group_num, n, k] (zero for a group without rows) */
} gg_op;

/*
 * Device-resident group sizes for every pass and input type: gg_prepare_device_lens's contract
 * (group_lens / group_offs in device memory, re-read by every gg_run, sizes that do not fit
 * reported by gg_plan_device_status) for the forward, dgrad and wgrad GEMMs, with 16-bit or fp8
 * inputs. a_dtype / b_dtype: equal GG_DTYPE_BF16 / GG_DTYPE_FP16, or fp8 (both e4m3, both e5m2,
 * or for dgrad / wgrad an e5m2 a with an e4m3 b), then out is bf16 scaled by a_scale[0] *
 * b_scale[g] (device floats; NULL for 16-bit types). Primus-Turbo passes group_lens_ptr /
 * group_offs_ptr to each of its grouped GEMMs (third_party/primus_turbo/include/primus_turbo/
 * grouped_gemm.h:35-36, 95-96, 112-130). total_m: rows of the row-indexed operands. The
 * requirements of the matching host-size entry point apply; wgrad's 2 GiB rule counts all
 * total_m rows, since any group may hold them all. wgrad always runs the per-tile variant here
 * (its K-step counts are not known on the host).
 */
int gg_prepare_device_lens_op(int op, int a_dtype, int b_dtype, int group_num, int64_t total_m, int64_t n,
                              int64_t k, const int64_t *group_lens, const int64_t *group_offs, const void *a,
                              const void *b, const float *a_scale, const float *b_scale, void *out,
                              void *stream, gg_plan **plan_out);

/*
 * Device-side size check of the last gg_run of a gg_prepare_device_lens plan, read back with a
 * synchronization of `stream`: GG_OK, or GG_ERR_INVALID naming the first group whose length or
 * offset was out of range (or a tile count beyond 32 bits, when nothing was computed).
 * *total_tiles (if not NULL) receives that run's tile count. For gg_prepare plans: GG_OK and
 * the plan's tile count, without a synchronization. No counterpart in the reference, which
 * does not check device-side sizes.
 */
int gg_plan_device_status(const gg_plan *plan, void *stream, int *total_tiles);

/*
 * offs[0] = 0, offs[g + 1] = offs[g] + lens[g] for g < group_num: the group offsets of
 * back-to-back groups, from device int64 lengths into device int64[group_num + 1], on `stream`
 * (one small launch, no sync). Replaces primus_turbo::compute_group_offs
 * (third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:138-140; its body is not
 * vendored, the semantics follow the group_offs_ptr contract of group_num + 1 first rows).
 */
int gg_compute_group_offs(const int64_t *group_lens, int64_t *group_offs, int group_num, void *stream);

/*
 * gg_prepare_device_lens_op + gg_run + gg_release in one call that allocates nothing. No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments,
 * rules and results as gg_prepare_device_lens_op followed by gg_run on `stream` (the current
 * device's); the launches are enqueued and the call returns without a sync.
 * The group table and its header live in a library-owned device array (scratch) of 131,328
 * bytes per GPU, held until the process ends: group_num is at most 8192 (else
 * GG_ERR_UNSUPPORTED, nothing launched). Every call on one GPU shares that array, so calls that
 * overlap on one GPU (other streams, other host threads) race on it; calls on one stream are
 * ordered. An empty contraction zero-fills the output with a kernel (no hipMemsetAsync). Sizes
 * found out of range on the device are not reported (their rows are not written): use a
 * gg_prepare_device_lens_op plan and gg_plan_device_status to check them. The first call on a
 * device looks up that device's scratch address and properties, so it must run outside stream
 * capture; later calls may be captured into a HIP graph (they launch kernels only, no
 * hipMemsetAsync).
 */
int gg_run_device_lens_noalloc(int op, int a_dtype, int b_dtype, int group_num, int64_t total_m, int64_t n,
                               int64_t k, const int64_t *group_lens, const int64_t *group_offs, const void *a,
                               const void *b, const float *a_scale, const float *b_scale, void *out,
                               void *stream);

/* Message of the last failed call on the calling thread ("" if none). */
const char *gg_last_error(void);

/*
 * Seeded N(0,1) fill of `count` elements of `dtype` at device pointer p, deterministic in
 * (seed, index). The benchmark input generator of bench/bench_main.cpp:160-176, 451-456
 * (splitmix64 + Box-Muller; seeds 1 for x, 2 for w). Harness helper, not part of the op.
 */
int gg_fill_randn(int dtype, void *p, size_t count, uint64_t seed, void *stream);

/*
 * Clock probe: enqueues one wave on `stream` that waits `seconds` (at most 10) of the device's
 * constant-rate wall clock and writes five uint64 to dev_out: the shader clock counter
 * (s_memtime) and the wall clock (s_memrealtime) at its start, the same two at its end, and the
 * wall clock's rate in Hz. Launched on a second stream beside a long run of gg_run, it gives the
 * run's effective shader clock, (end - start cycles) / (end - start ticks) * rate. It uses a few
 * VGPRs and no LDS, so it runs next to a GEMM workgroup. Measurement helper, not part of the op;
 * the reference samples the clock with amd-smi instead (scripts/power.py:1-9).
 */
int gg_clock_probe(uint64_t *dev_out, double seconds, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GG_GROUPED_GEMM_H */
