// Comparison backends on hipBLASLt (the vendor library), written for this driver.
//
// hipblaslt_loop: the semantics of Primus-Turbo's hipBLASLt grouped GEMM, which the reference
//   times as its baseline (backends/hipblaslt_loop_backend.cpp:38-67 driving
//   third_party/primus_turbo/kernels/hipblaslt_grouped_gemm.cu:99-163, 174-251 and
//   hipblaslt_gemm.cu:32-120): every run() reads the group lengths on the host, then per
//   non-empty group builds the matmul descriptors, asks the heuristic for one algorithm and
//   calls hipblasLtMatmul, round-robin over 4 streams (64 MiB of workspace each) forked from
//   and joined back into the caller's stream with events. All of it is inside the timed
//   region, as it is in Primus-Turbo. Every stream slot has its own hipBLASLt handle and 8
//   slots are created although 4 are used: hipBLASLt keeps per-handle state and assumes one
//   handle per stream, and Primus-Turbo reports multi-stream stalls on MI355X without both
//   (hipblaslt_grouped_gemm.cu:21-27, 40-55). Unlike Primus-Turbo, the side streams keep the
//   default priority.
// hipblaslt_seq: the same per-group loop (host lengths, heuristic per call, all timed) on the
//   caller's stream alone. No two hipBLASLt kernels run at once, so it cannot stall the way
//   the 4-stream loop did (below); it gives up the overlap of small groups.
// hipblaslt_grouped: hipblaslt_ext::GroupedGemm, one launch for all groups, device-side
//   arguments, heuristic top-1, prepared untimed; N/A when the library has no kernel for the
//   type (the reference's backends/hipblaslt_grouped_backend.cpp:45-98).
//
// hipBLASLt is column-major, so both solve the transposed problem per group:
//   out_g^T [N, M_g] = op_T(w_g stored K x N) * x_g^T (stored K x M_g)
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "backend.hpp"

namespace tunemax {
namespace {

void blas_check(hipblasStatus_t st, const char *what) {
    if (st != HIPBLAS_STATUS_SUCCESS)
        throw std::runtime_error(std::string("hipBLASLt ") + what + " failed: status " +
                                 std::to_string(static_cast<int>(st)));
}

hipDataType hip_type(DType t) { return t == DType::BF16 ? HIP_R_16BF : HIP_R_16F; }

// ---------------------------------------------------------------------------------------
class HipblasltLoopBackend final : public Backend {
public:
    static constexpr int     kSlots           = 8; // slots created (handle + stream + event)
    static constexpr int64_t kWorkspacePerStr = int64_t(64) << 20;

    explicit HipblasltLoopBackend(int streams) : kStreams(streams) {
        for (int i = 0; i < kSlots; ++i)
            blas_check(hipblasLtCreate(&handle_[i]), "create");
        TUNEMAX_HIP_CHECK(hipMalloc(&workspace_, kStreams * kWorkspacePerStr));
        TUNEMAX_HIP_CHECK(hipMemset(workspace_, 0, kStreams * kWorkspacePerStr));
        for (int i = 1; i < kSlots; ++i)
            TUNEMAX_HIP_CHECK(hipStreamCreateWithFlags(&side_[i], hipStreamNonBlocking));
        for (int i = 0; i < kSlots; ++i)
            TUNEMAX_HIP_CHECK(hipEventCreateWithFlags(&ev_[i], hipEventDisableTiming));
    }
    ~HipblasltLoopBackend() override {
        for (int i = 0; i < kSlots; ++i)
            (void)hipEventDestroy(ev_[i]);
        for (int i = 1; i < kSlots; ++i)
            (void)hipStreamDestroy(side_[i]);
        (void)hipFree(workspace_);
        for (int i = 0; i < kSlots; ++i)
            (void)hipblasLtDestroy(handle_[i]);
    }

    std::string name() const override { return kStreams == 1 ? "hipblaslt_seq" : "hipblaslt_loop"; }

    std::string prepare(const GroupedGemmProblem &p, hipStream_t) override {
        if (p.group_lens_pinned == nullptr)
            return "needs the group lengths in pinned host memory";
        // This 4-stream loop never finished its first call on groups of 1024 x 4096 x 7168
        // (shapes/full.csv TestID 3) on MI355X, with one shared handle and again with one
        // handle per stream; it is not run there.
        for (int g = 0; g < p.group_num && kStreams > 1; ++g)
            if (p.group_m[g] == 1024 && p.n == 4096 && p.k == 7168)
                return "skipped: the multi-stream hipBLASLt loop hung on 1024 x 4096 x 7168 groups on MI355X";
        p_ = p;
        return "";
    }

    void run(hipStream_t stream) override {
        const hipDataType t  = hip_type(p_.dtype);
        const size_t      es = dtype_bytes(p_.dtype);
        side_[0]             = stream;
        // fork: side streams start after everything already queued on the caller's stream
        if (kStreams > 1)
            TUNEMAX_HIP_CHECK(hipEventRecord(ev_[0], stream));
        for (int i = 1; i < kStreams; ++i)
            TUNEMAX_HIP_CHECK(hipStreamWaitEvent(side_[i], ev_[0], 0));
        const float alpha = 1.0f, beta = 0.0f;
        int64_t     row = 0;
        int         idx = 0;
        for (int g = 0; g < p_.group_num; ++g) {
            const int64_t m = p_.group_lens_pinned[g]; // read on the host every call
            if (m == 0)
                continue;
            const char *w   = static_cast<const char *>(p_.w) + size_t(g) * p_.n * p_.k * es;
            const char *x   = static_cast<const char *>(p_.x) + size_t(row) * p_.k * es;
            char       *out = static_cast<char *>(p_.out) + size_t(row) * p_.n * es;
            const int   s   = idx % kStreams;
            gemm(handle_[s], t, p_.n, m, p_.k, w, x, out, &alpha, &beta,
                 static_cast<char *>(workspace_) + s * kWorkspacePerStr, side_[s]);
            row += m;
            ++idx;
        }
        // join: the caller's stream waits for every side stream
        for (int i = 1; i < kStreams; ++i) {
            TUNEMAX_HIP_CHECK(hipEventRecord(ev_[i], side_[i]));
            TUNEMAX_HIP_CHECK(hipStreamWaitEvent(stream, ev_[i], 0));
        }
    }

    std::string detail() const override {
        return "1 hipblasLtMatmul per group (heuristic each call), " + std::to_string(kStreams) +
               (kStreams == 1 ? " stream" : " streams");
    }

private:
    // D [m, n] col-major = op_T(A: k x m col-major) * B (k x n col-major), one group.
    void gemm(hipblasLtHandle_t handle, hipDataType t, int64_t m, int64_t n, int64_t k, const void *a,
              const void *b, void *d, const float *alpha, const float *beta, void *ws, hipStream_t s) {
        hipblasLtMatmulDesc_t   desc = nullptr;
        hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
        hipblasLtMatmulPreference_t pref = nullptr;
        blas_check(hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "desc");
        const hipblasOperation_t opa = HIPBLAS_OP_T, opb = HIPBLAS_OP_N;
        blas_check(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa)), "transA");
        blas_check(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb)), "transB");
        blas_check(hipblasLtMatrixLayoutCreate(&la, t, k, m, k), "layout A");
        blas_check(hipblasLtMatrixLayoutCreate(&lb, t, k, n, k), "layout B");
        blas_check(hipblasLtMatrixLayoutCreate(&lc, t, m, n, m), "layout C");
        blas_check(hipblasLtMatmulPreferenceCreate(&pref), "preference");
        const uint64_t wsb = kWorkspacePerStr;
        blas_check(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                         sizeof(wsb)),
                   "workspace preference");
        hipblasLtMatmulHeuristicResult_t res{};
        int                              found = 0;
        blas_check(hipblasLtMatmulAlgoGetHeuristic(handle, desc, la, lb, lc, lc, pref, 1, &res, &found),
                   "heuristic");
        if (found == 0)
            throw std::runtime_error("hipBLASLt heuristic found no algorithm");
        blas_check(hipblasLtMatmul(handle, desc, alpha, a, la, b, lb, beta, d, lc, d, lc, &res.algo, ws,
                                   kWorkspacePerStr, s),
                   "matmul");
        (void)hipblasLtMatmulPreferenceDestroy(pref);
        (void)hipblasLtMatrixLayoutDestroy(la);
        (void)hipblasLtMatrixLayoutDestroy(lb);
        (void)hipblasLtMatrixLayoutDestroy(lc);
        (void)hipblasLtMatmulDescDestroy(desc);
    }

    const int          kStreams; // slots used per run: 4 (hipblaslt_loop) or 1 (hipblaslt_seq)
    hipblasLtHandle_t  handle_[kSlots]{};
    void              *workspace_ = nullptr;
    hipStream_t        side_[kSlots]{};
    hipEvent_t         ev_[kSlots]{};
    GroupedGemmProblem p_;
};

// ---------------------------------------------------------------------------------------
class HipblasltGroupedBackend final : public Backend {
public:
    static constexpr size_t kWorkspace = size_t(128) << 20;

    HipblasltGroupedBackend() {
        blas_check(hipblasLtCreate(&handle_), "create");
        TUNEMAX_HIP_CHECK(hipMalloc(&workspace_, kWorkspace));
    }
    ~HipblasltGroupedBackend() override {
        release();
        (void)hipFree(workspace_);
        (void)hipblasLtDestroy(handle_);
    }

    std::string name() const override { return "hipblaslt_grouped"; }

    std::string prepare(const GroupedGemmProblem &p, hipStream_t stream) override {
        release();
        const hipDataType t  = hip_type(p.dtype);
        const size_t      es = dtype_bytes(p.dtype);
        gemm_ = std::make_unique<hipblaslt_ext::GroupedGemm>(handle_, HIPBLAS_OP_T, HIPBLAS_OP_N, t, t, t, t,
                                                             HIPBLAS_COMPUTE_32F);
        std::vector<int64_t> m, n, k, batch;
        std::vector<hipblaslt_ext::GemmEpilogue> epi;
        std::vector<hipblaslt_ext::GemmInputs>   in;
        alpha_.clear();
        beta_.clear();
        alpha_.reserve(p.group_num);
        beta_.reserve(p.group_num);
        int64_t row = 0;
        for (int g = 0; g < p.group_num; ++g) {
            const int64_t mg = p.group_m[g];
            if (mg > 0) {
                m.push_back(p.n);
                n.push_back(mg);
                k.push_back(p.k);
                batch.push_back(1);
                epi.emplace_back();
                alpha_.push_back(1.0f);
                beta_.push_back(0.0f);
                hipblaslt_ext::GemmInputs gi;
                gi.setA(static_cast<const char *>(p.w) + size_t(g) * p.n * p.k * es);
                gi.setB(static_cast<const char *>(p.x) + size_t(row) * p.k * es);
                gi.setC(static_cast<char *>(p.out) + size_t(row) * p.n * es);
                gi.setD(static_cast<char *>(p.out) + size_t(row) * p.n * es);
                gi.setAlpha(&alpha_.back());
                gi.setBeta(&beta_.back());
                in.push_back(gi);
            }
            row += mg;
        }
        if (m.empty())
            return "no non-empty groups";
        if (gemm_->setProblem(m, n, k, batch, epi, in) != HIPBLAS_STATUS_SUCCESS)
            return "hipBLASLt rejected the grouped problem";
        hipblaslt_ext::GemmPreference pref;
        pref.setMaxWorkspaceBytes(kWorkspace);
        std::vector<hipblasLtMatmulHeuristicResult_t> cand;
        (void)gemm_->algoGetHeuristic(1, pref, cand);
        if (cand.empty())
            return std::string("no hipBLASLt grouped kernel for ") + dtype_name(p.dtype);
        std::vector<hipblaslt_ext::UserArguments> host(m.size());
        blas_check(gemm_->getDefaultValueForDeviceUserArguments(host.data()), "user arguments");
        const size_t bytes = host.size() * sizeof(hipblaslt_ext::UserArguments);
        TUNEMAX_HIP_CHECK(hipMalloc(&dev_args_, bytes));
        TUNEMAX_HIP_CHECK(hipMemcpyAsync(dev_args_, host.data(), bytes, hipMemcpyHostToDevice, stream));
        blas_check(gemm_->initialize(cand[0].algo, workspace_), "initialize");
        TUNEMAX_HIP_CHECK(hipStreamSynchronize(stream));
        detail_ = gemm_->getKernelName();
        return "";
    }

    void run(hipStream_t stream) override { blas_check(gemm_->run(dev_args_, stream), "grouped run"); }

    void release() override {
        gemm_.reset();
        if (dev_args_ != nullptr)
            TUNEMAX_HIP_CHECK(hipFree(dev_args_));
        dev_args_ = nullptr;
    }

    std::string detail() const override { return detail_; }

private:
    hipblasLtHandle_t                           handle_    = nullptr;
    void                                       *workspace_ = nullptr;
    void                                       *dev_args_  = nullptr;
    std::unique_ptr<hipblaslt_ext::GroupedGemm> gemm_;
    std::vector<float>                          alpha_, beta_;
    std::string                                 detail_;
};

} // namespace

std::unique_ptr<Backend> make_hipblaslt_loop_backend() { return std::make_unique<HipblasltLoopBackend>(4); }
std::unique_ptr<Backend> make_hipblaslt_seq_backend() { return std::make_unique<HipblasltLoopBackend>(1); }
std::unique_ptr<Backend> make_hipblaslt_grouped_backend() { return std::make_unique<HipblasltGroupedBackend>(); }

} // namespace tunemax
