// Grouped-GEMM backend interface, source-compatible with the reference's
// common/backend.hpp:15-83 (same names, fields and call contract), so driver code written
// against that header compiles against this one; the only new line a driver needs is the
// factory of the backend it wants.
//
// Contract (unchanged): prepare() is untimed and returns "" or a reason the backend cannot
// run the problem (reported as N/A); run() is timed and enqueues exactly one grouped GEMM on
// the stream without synchronizing; release() frees what prepare() allocated.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

// Print the failing HIP call and exit (the reference's error convention for its driver;
// the library under it returns status codes instead).
#define TUNEMAX_HIP_CHECK(expr)                                                                   \
    do {                                                                                          \
        const hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) {                                                                   \
            std::fprintf(stderr, "HIP error %s at %s:%d: %s\n", hipGetErrorString(e_), __FILE__,  \
                         __LINE__, #expr);                                                        \
            std::exit(1);                                                                         \
        }                                                                                         \
    } while (0)

namespace tunemax {

enum class DType { BF16, FP16 };

inline const char *dtype_name(DType t) { return t == DType::BF16 ? "bf16" : "fp16"; }
inline size_t      dtype_bytes(DType) { return 2; }

// out[rows of group g] = x[rows of group g] @ w[g]^T with
//   x [sum(group_m), k], w [group_num, n, k], out [sum(group_m), n], all row-major,
// fp32 accumulation, output in the input type.
struct GroupedGemmProblem {
    DType                dtype     = DType::BF16;
    int                  group_num = 0;
    int64_t              n         = 0;
    int64_t              k         = 0;
    std::vector<int64_t> group_m; // host, one per group

    const void *x   = nullptr; // device
    const void *w   = nullptr; // device
    void       *out = nullptr; // device

    // The same lengths in pinned host memory (the per-group loop backend reads them on the
    // host every call, as Primus-Turbo does).
    const int64_t *group_lens_pinned = nullptr;

    int64_t total_m() const {
        int64_t s = 0;
        for (const int64_t m : group_m)
            s += m;
        return s;
    }
    double flops() const { return 2.0 * double(total_m()) * double(n) * double(k); }
};

class Backend {
public:
    virtual ~Backend()                                                                 = default;
    virtual std::string name() const                                                   = 0;
    virtual std::string prepare(const GroupedGemmProblem &problem, hipStream_t stream) = 0;
    virtual void        run(hipStream_t stream)                                        = 0;
    virtual void        release() {}
    virtual std::string detail() const { return ""; }
};

// The MI355X persistent grouped GEMM of this repository (over include/gg_grouped_gemm.h).
std::unique_ptr<Backend> make_mi355x_backend();
// hipBLASLt's own grouped GEMM (hipblaslt_ext::GroupedGemm, heuristic top-1).
std::unique_ptr<Backend> make_hipblaslt_grouped_backend();
// One hipblasLtMatmul per group with a heuristic query each, over 4 streams (the
// Primus-Turbo loop the reference compares against).
std::unique_ptr<Backend> make_hipblaslt_loop_backend();
// The same loop on the caller's stream only (no concurrent hipBLASLt kernels).
std::unique_ptr<Backend> make_hipblaslt_seq_backend();

// Name -> factory, for drivers (the reference hard-codes an if-chain,
// bench/bench_main.cpp:398-407).
inline const std::map<std::string, std::function<std::unique_ptr<Backend>()>> &backend_registry() {
    static const std::map<std::string, std::function<std::unique_ptr<Backend>()>> r = {
        {"mi355x", make_mi355x_backend},
        {"hipblaslt_grouped", make_hipblaslt_grouped_backend},
        {"hipblaslt_loop", make_hipblaslt_loop_backend},
        {"hipblaslt_seq", make_hipblaslt_seq_backend},
    };
    return r;
}

} // namespace tunemax
