// Comparison backends on hipBLASLt, the vendor library, for this repository's drivers (gg_bench,
// and bench.py through the C shim in gg_compare.cpp). They are what the reference measures its
// kernel against (README.md:54-58); nothing on the product path uses them.
//
//   hipblaslt_loop     Primus-Turbo's cost model (backends/hipblaslt_loop_backend.cpp:38-67 over
//                      third_party/primus_turbo/kernels/hipblaslt_grouped_gemm.cu:99-163, 174-251):
//                      every run() reads the group lengths on the host and, per non-empty group,
//                      builds the matmul descriptors, asks the heuristic for one algorithm and calls
//                      hipblasLtMatmul; groups go round-robin over 4 streams forked from and joined
//                      into the caller's stream. All of it is inside the timed region.
//   hipblaslt_seq      the same per-group work on the caller's stream only.
//   hipblaslt_grouped  hipblaslt_ext::GroupedGemm: one launch for all groups, arguments in device
//                      memory, heuristic top-1, set up in prepare() (the reference's
//                      backends/hipblaslt_grouped_backend.cpp:45-98).
//
// Stream-K in the 4-stream loop. A hipBLASLt stream-K kernel (Tensile "SK" solutions) launches
// a grid sized for the whole GPU, and the workgroup that owns a split tile waits in a loop for
// flags that the workgroups computing the tile's other K ranges set in the workspace. That wait
// ends only if those workgroups get a CU, which the kernel is sure of only when it has the GPU to
// itself. Four such kernels on four streams split the CUs between them, and each can fill its
// share with workgroups that wait for ones still queued behind them: none of the four finishes.
// Primus-Turbo runs the heuristic's first choice on 4 streams, and that loop hung on its first
// call for 8 groups of 1024 x 4096 x 7168 (shapes/full.csv TestID 3) while the same kernels one
// at a time (hipblaslt_seq) finished all 360 cases. The installed hipBLASLt's heuristic ranks
// only stream-K kernels (SK3) in its first 64 results for every bf16 and fp16 shape tried on
// MI355X, while the library holds about 45 other kernels that support each shape (all
// getAllAlgos results that pass matmulIsAlgoSupported within the workspace limit and are not
// stream-K). So the 4-stream mode, per distinct group size, times each of those kernels once in
// prepare() (one untimed launch, then two timed ones, on the problem's own inputs, into a scratch
// output so that the driver's cleared output stays cleared) and keeps the fastest. run() keeps
// Primus-Turbo's per-call work, the heuristic query included, and launches the heuristic's first
// choice unless it is stream-K, in which case it launches the kept kernel after checking it
// against the call's descriptors (matmulIsAlgoSupported). No stream-K kernel ever runs on the 4
// streams; hipblaslt_seq keeps the heuristic's first choice, stream-K or not.
//
// Failures of HIP or hipBLASLt calls throw std::runtime_error (the driver's ERROR row, a Python
// exception through the shim); nothing here exits the process. Streams keep the default priority.
//
// hipBLASLt is column-major; each group is solved transposed:
//   out_g^T [N x M_g, ld N] = op_T(w_g: K x N col-major, ld K) * (x_g: K x M_g col-major, ld K)
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <cctype>
#include <map>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include "backend.hpp"
#include "gg_compare.h"

namespace tunemax {
namespace {

void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void lt_ok(hipblasStatus_t s, const char *what) {
    if (s != HIPBLAS_STATUS_SUCCESS)
        throw std::runtime_error(std::string("hipBLASLt ") + what + ": status " + std::to_string(int(s)));
}

hipDataType lt_type(DType t) { return t == DType::BF16 ? HIP_R_16BF : HIP_R_16F; }

constexpr uint64_t kLoopWorkspace = uint64_t(64) << 20; // per stream slot

// The descriptors of one group's matmul (out^T = op_T(w) * x^T), released on scope exit.
class GroupMatmul {
public:
    GroupMatmul(hipDataType t, int64_t n, int64_t m_g, int64_t k, uint64_t ws_bytes) {
        lt_ok(hipblasLtMatmulDescCreate(&op_, HIPBLAS_COMPUTE_32F, HIP_R_32F), "matmul descriptor");
        const hipblasOperation_t trans = HIPBLAS_OP_T, keep = HIPBLAS_OP_N;
        lt_ok(hipblasLtMatmulDescSetAttribute(op_, HIPBLASLT_MATMUL_DESC_TRANSA, &trans, sizeof(trans)), "op A");
        lt_ok(hipblasLtMatmulDescSetAttribute(op_, HIPBLASLT_MATMUL_DESC_TRANSB, &keep, sizeof(keep)), "op B");
        lt_ok(hipblasLtMatrixLayoutCreate(&w_, t, k, n, k), "w layout");
        lt_ok(hipblasLtMatrixLayoutCreate(&x_, t, k, m_g, k), "x layout");
        lt_ok(hipblasLtMatrixLayoutCreate(&out_, t, n, m_g, n), "out layout");
        lt_ok(hipblasLtMatmulPreferenceCreate(&pref_), "preference");
        lt_ok(hipblasLtMatmulPreferenceSetAttribute(pref_, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws_bytes,
                                                    sizeof(ws_bytes)),
              "workspace limit");
        ws_bytes_ = ws_bytes;
    }
    GroupMatmul(const GroupMatmul &)            = delete;
    GroupMatmul &operator=(const GroupMatmul &) = delete;
    ~GroupMatmul() {
        (void)hipblasLtMatmulPreferenceDestroy(pref_);
        (void)hipblasLtMatrixLayoutDestroy(out_);
        (void)hipblasLtMatrixLayoutDestroy(x_);
        (void)hipblasLtMatrixLayoutDestroy(w_);
        (void)hipblasLtMatmulDescDestroy(op_);
    }

    // The heuristic's first choice.
    hipblasLtMatmulHeuristicResult_t choose(hipblasLtHandle_t h) const {
        hipblasLtMatmulHeuristicResult_t best{};
        int                              n = 0;
        lt_ok(hipblasLtMatmulAlgoGetHeuristic(h, op_, w_, x_, out_, out_, pref_, 1, &best, &n), "heuristic");
        if (n == 0)
            throw std::runtime_error("hipBLASLt has no algorithm for this group");
        return best;
    }

    // Whether `algo` solves this matmul within the workspace limit (matmulIsAlgoSupported, which
    // also records the problem in the algo, as hipblasLtMatmul expects).
    bool supports(hipblasLtHandle_t h, hipblasLtMatmulAlgo_t &algo) const {
        const float one = 1.0f, zero = 0.0f;
        size_t      need = 0;
        return hipblaslt_ext::matmulIsAlgoSupported(h, op_, &one, w_, x_, &zero, out_, out_, algo, need) ==
                   HIPBLAS_STATUS_SUCCESS &&
               need <= ws_bytes_;
    }

    void launch(hipblasLtHandle_t h, const hipblasLtMatmulAlgo_t &algo, const void *w, const void *x, void *out,
                void *ws, hipStream_t s) const {
        const float one = 1.0f, zero = 0.0f;
        lt_ok(hipblasLtMatmul(h, op_, &one, w, w_, x, x_, &zero, out, out_, out, out_, &algo, ws, ws_bytes_, s),
              "matmul");
    }

private:
    hipblasLtMatmulDesc_t       op_   = nullptr;
    hipblasLtMatrixLayout_t     w_    = nullptr;
    hipblasLtMatrixLayout_t     x_    = nullptr;
    hipblasLtMatrixLayout_t     out_  = nullptr;
    hipblasLtMatmulPreference_t pref_ = nullptr;
    uint64_t                    ws_bytes_ = 0;
};

// Tensile names a stream-K solution with the token "_SK<n>_", n > 0.
bool stream_k_kernel(const std::string &name) {
    for (size_t p = name.find("_SK"); p != std::string::npos; p = name.find("_SK", p + 1)) {
        size_t q = p + 3;
        while (q < name.size() && std::isdigit(static_cast<unsigned char>(name[q])))
            ++q;
        if (q > p + 3 && (q == name.size() || name[q] == '_') && std::stoi(name.substr(p + 3, q - p - 3)) > 0)
            return true;
    }
    return false;
}

// ---------------------------------------------------------------------------------------
// hipblaslt_loop / hipblaslt_seq
// ---------------------------------------------------------------------------------------
class PerGroupLoop final : public Backend {
public:
    // streams: 4 (hipblaslt_loop) or 1 (hipblaslt_seq). The 4-stream mode keeps 8 handle slots,
    // as Primus-Turbo does (hipblaslt_grouped_gemm.cu:21-27: 8 slots, 4 used).
    explicit PerGroupLoop(int streams) : streams_(streams), slots_(streams > 1 ? 8 : 1) {
        handles_.assign(size_t(slots_), nullptr);
        side_.assign(size_t(slots_), nullptr);
        joined_.assign(size_t(slots_), nullptr);
        for (auto &h : handles_)
            lt_ok(hipblasLtCreate(&h), "create handle");
        for (int i = 1; i < slots_; ++i)
            hip_ok(hipStreamCreateWithFlags(&side_[size_t(i)], hipStreamNonBlocking), "side stream");
        for (auto &e : joined_)
            hip_ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "event");
        hip_ok(hipMalloc(&workspace_, size_t(streams_) * kLoopWorkspace), "workspace");
        // stream-K kernels keep their flags in the workspace and expect zeros at the start
        hip_ok(hipMemset(workspace_, 0, size_t(streams_) * kLoopWorkspace), "workspace clear");
    }
    ~PerGroupLoop() override {
        (void)hipFree(workspace_);
        for (auto e : joined_)
            (void)hipEventDestroy(e);
        for (size_t i = 1; i < side_.size(); ++i)
            (void)hipStreamDestroy(side_[i]);
        for (auto h : handles_)
            (void)hipblasLtDestroy(h);
    }

    std::string name() const override { return streams_ > 1 ? "hipblaslt_loop" : "hipblaslt_seq"; }

    std::string prepare(const GroupedGemmProblem &p, hipStream_t stream) override {
        if (p.group_lens_pinned == nullptr)
            return "needs the group lengths in pinned host memory";
        if (int64_t(p.group_m.size()) != p.group_num)
            throw std::runtime_error("group_m has " + std::to_string(p.group_m.size()) + " entries for " +
                                     std::to_string(p.group_num) + " groups");
        problem_ = p;
        kernels_.clear();
        picks_.clear();
        std::set<int64_t> sizes(p.group_m.begin(), p.group_m.end());
        for (const int64_t m : sizes) {
            if (m <= 0)
                continue;
            const GroupMatmul                      mm(lt_type(p.dtype), p.n, m, p.k, kLoopWorkspace);
            const hipblasLtMatmulHeuristicResult_t first = mm.choose(handles_[0]);
            hipblasLtMatmulAlgo_t                  algo  = first.algo;
            std::string kn = hipblaslt_ext::getKernelNameFromAlgo(handles_[0], algo);
            Pick        pick{hipblaslt_ext::getIndexFromAlgo(algo), false, first.algo};
            if (streams_ > 1 && stream_k_kernel(kn)) {
                std::string why;
                if (!fastest_without_stream_k(p, m, mm, stream, &pick.kept, &kn, &why))
                    return "N/A: no hipBLASLt kernel other than stream-K supports groups of " + std::to_string(m) +
                           " rows (" + why + "), and stream-K kernels on " + std::to_string(streams_) +
                           " streams at once can deadlock (each waits on workgroups that need the whole GPU)";
                pick.replaced = true;
                kn += " (timed pick: the heuristic's first choice is stream-K)";
            }
            picks_[m] = pick;
            kernels_ += (kernels_.empty() ? "" : "; ") + kn;
        }
        return "";
    }

    void run(hipStream_t stream) override {
        const GroupedGemmProblem &p  = problem_;
        const size_t              es = dtype_bytes(p.dtype);
        const hipDataType         t  = lt_type(p.dtype);
        if (streams_ > 1) { // fork: the side streams start after the caller's queued work
            hip_ok(hipEventRecord(joined_[0], stream), "fork event");
            for (int i = 1; i < streams_; ++i)
                hip_ok(hipStreamWaitEvent(side_[size_t(i)], joined_[0], 0), "fork wait");
        }
        int64_t row  = 0;
        int     used = 0;
        for (int g = 0; g < p.group_num; ++g) {
            const int64_t m = p.group_lens_pinned[g]; // read on the host each call
            if (m <= 0)
                continue;
            const int                        s  = used++ % streams_;
            const hipStream_t                st = s == 0 ? stream : side_[size_t(s)];
            const hipblasLtHandle_t          h  = handles_[size_t(s)];
            const GroupMatmul                mm(t, p.n, m, p.k, kLoopWorkspace);
            hipblasLtMatmulHeuristicResult_t pick = mm.choose(h); // the heuristic, every call
            if (streams_ > 1) {
                // a stream-K first choice never runs on the 4 streams: the kernel timed in
                // prepare() for this group size replaces it
                const auto it = picks_.find(m);
                if (it == picks_.end())
                    throw std::runtime_error("group of " + std::to_string(m) + " rows: sizes changed since prepare()");
                if (hipblaslt_ext::getIndexFromAlgo(pick.algo) != it->second.first_index &&
                    stream_k_kernel(hipblaslt_ext::getKernelNameFromAlgo(h, pick.algo)))
                    throw std::runtime_error("the heuristic changed its stream-K choice since prepare()");
                if (it->second.replaced) {
                    pick.algo = it->second.kept;
                    if (!mm.supports(h, pick.algo))
                        throw std::runtime_error("the kept kernel no longer supports the group");
                }
            }
            mm.launch(h, pick.algo, static_cast<const char *>(p.w) + size_t(g) * p.n * p.k * es,
                      static_cast<const char *>(p.x) + size_t(row) * p.k * es,
                      static_cast<char *>(p.out) + size_t(row) * p.n * es,
                      static_cast<char *>(workspace_) + size_t(s) * kLoopWorkspace, st);
            row += m;
        }
        for (int i = 1; i < streams_; ++i) { // join into the caller's stream
            hip_ok(hipEventRecord(joined_[size_t(i)], side_[size_t(i)]), "join event");
            hip_ok(hipStreamWaitEvent(stream, joined_[size_t(i)], 0), "join wait");
        }
    }

    std::string detail() const override {
        return "hipblasLtMatmul per group, heuristic each call, " + std::to_string(streams_) +
               (streams_ > 1 ? " streams, no stream-K" : " stream") + (kernels_.empty() ? "" : " [" + kernels_ + "]");
    }

private:
    // Per group size: the heuristic's first choice (its solution index) and, when that is
    // stream-K, the kernel that replaces it on the 4 streams.
    struct Pick {
        int                   first_index = -1;
        bool                  replaced    = false;
        hipblasLtMatmulAlgo_t kept{};
    };

    // The fastest kernel that is not stream-K among all the library's kernels that support one
    // group of m rows within the workspace limit: each is launched once untimed and twice timed
    // on the caller's stream, reading the problem's x and w (group 0's rows and weights) and
    // writing a scratch output. False (with *why) if none supports the group or every launch fails.
    bool fastest_without_stream_k(const GroupedGemmProblem &p, int64_t m, const GroupMatmul &mm, hipStream_t stream,
                                  hipblasLtMatmulAlgo_t *best, std::string *name, std::string *why) {
        const hipDataType t = lt_type(p.dtype);
        auto             &all = all_algos_[int(t)];
        if (all.empty())
            lt_ok(hipblaslt_ext::getAllAlgos(handles_[0], hipblaslt_ext::GemmType::HIPBLASLT_GEMM, HIPBLAS_OP_T,
                                             HIPBLAS_OP_N, t, t, t, t, HIPBLAS_COMPUTE_32F, all),
                  "all algorithms");
        std::vector<hipblasLtMatmulAlgo_t> cand;
        for (const auto &r : all) {
            hipblasLtMatmulAlgo_t a = r.algo;
            if (mm.supports(handles_[0], a) && !stream_k_kernel(hipblaslt_ext::getKernelNameFromAlgo(handles_[0], a)))
                cand.push_back(a);
        }
        if (cand.empty()) {
            *why = std::to_string(all.size()) + " kernels checked";
            return false;
        }
        const size_t es   = dtype_bytes(p.dtype);
        void        *out  = nullptr;
        hipEvent_t   e[2] = {nullptr, nullptr};
        hip_ok(hipMalloc(&out, size_t(m) * size_t(p.n) * es), "scratch output");
        float best_ms = -1.0f;
        try {
            for (auto &ev : e)
                hip_ok(hipEventCreate(&ev), "timing event");
            for (auto &a : cand) {
                try {
                    mm.launch(handles_[0], a, p.w, p.x, out, workspace_, stream);
                    hip_ok(hipEventRecord(e[0], stream), "timing event");
                    for (int r = 0; r < 2; ++r)
                        mm.launch(handles_[0], a, p.w, p.x, out, workspace_, stream);
                    hip_ok(hipEventRecord(e[1], stream), "timing event");
                    hip_ok(hipEventSynchronize(e[1]), "timing sync");
                } catch (const std::runtime_error &) {
                    hip_ok(hipStreamSynchronize(stream), "timing sync");
                    continue; // a kernel that fails to launch is not a candidate
                }
                float ms = 0.0f;
                hip_ok(hipEventElapsedTime(&ms, e[0], e[1]), "timing");
                if (best_ms < 0.0f || ms < best_ms) {
                    best_ms = ms;
                    *best   = a;
                }
            }
        } catch (...) {
            for (auto ev : e)
                if (ev != nullptr)
                    (void)hipEventDestroy(ev);
            (void)hipFree(out);
            throw;
        }
        for (auto ev : e)
            (void)hipEventDestroy(ev);
        hip_ok(hipFree(out), "scratch output");
        if (best_ms < 0.0f) {
            *why = std::to_string(cand.size()) + " candidates failed to launch";
            return false;
        }
        *name = hipblaslt_ext::getKernelNameFromAlgo(handles_[0], *best) + ", fastest of " + std::to_string(cand.size()) +
                " non-stream-K kernels (" + std::to_string(best_ms / 2.0f) + " ms)";
        return true;
    }

    const int                      streams_;
    const int                      slots_;
    std::vector<hipblasLtHandle_t> handles_;
    std::vector<hipStream_t>       side_;   // [0] unused: slot 0 is the caller's stream
    std::vector<hipEvent_t>        joined_; // [0] the fork point, [i] side stream i done
    void                          *workspace_ = nullptr;
    GroupedGemmProblem             problem_;
    std::string                    kernels_;
    std::map<int64_t, Pick>        picks_;     // per group size (4-stream mode)
    std::map<int, std::vector<hipblasLtMatmulHeuristicResult_t>> all_algos_; // getAllAlgos, per data type
};

// ---------------------------------------------------------------------------------------
// hipblaslt_grouped
// ---------------------------------------------------------------------------------------
class LtGrouped final : public Backend {
public:
    static constexpr size_t kWorkspace = size_t(128) << 20;

    LtGrouped() {
        lt_ok(hipblasLtCreate(&handle_), "create handle");
        hip_ok(hipMalloc(&workspace_, kWorkspace), "workspace");
    }
    ~LtGrouped() override {
        release();
        (void)hipFree(workspace_);
        (void)hipblasLtDestroy(handle_);
    }

    std::string name() const override { return "hipblaslt_grouped"; }

    std::string prepare(const GroupedGemmProblem &p, hipStream_t stream) override {
        release();
        if (int64_t(p.group_m.size()) != p.group_num)
            throw std::runtime_error("group_m does not hold group_num entries");
        const hipDataType t  = lt_type(p.dtype);
        const size_t      es = dtype_bytes(p.dtype);
        // one entry per non-empty group: sizes in column-major terms, pointers, alpha / beta
        std::vector<int64_t>                     rows, cols, depth, batch;
        std::vector<hipblaslt_ext::GemmEpilogue> epilogue;
        std::vector<hipblaslt_ext::GemmInputs>   inputs;
        scalars_.assign(size_t(2 * p.group_num), 0.0f);
        int64_t row = 0;
        for (int g = 0; g < p.group_num; ++g) {
            const int64_t m = p.group_m[size_t(g)];
            if (m > 0) {
                rows.push_back(p.n);
                cols.push_back(m);
                depth.push_back(p.k);
                batch.push_back(1);
                epilogue.emplace_back();
                float *ab = &scalars_[size_t(2 * g)];
                ab[0]     = 1.0f; // alpha; ab[1] = beta = 0
                void *o   = static_cast<char *>(p.out) + size_t(row) * p.n * es;
                hipblaslt_ext::GemmInputs in;
                in.setA(static_cast<const char *>(p.w) + size_t(g) * p.n * p.k * es);
                in.setB(static_cast<const char *>(p.x) + size_t(row) * p.k * es);
                in.setC(o);
                in.setD(o);
                in.setAlpha(ab);
                in.setBeta(ab + 1);
                inputs.push_back(in);
            }
            row += m;
        }
        if (rows.empty())
            return "no non-empty groups";
        op_ = std::make_unique<hipblaslt_ext::GroupedGemm>(handle_, HIPBLAS_OP_T, HIPBLAS_OP_N, t, t, t, t,
                                                          HIPBLAS_COMPUTE_32F);
        if (op_->setProblem(rows, cols, depth, batch, epilogue, inputs) != HIPBLAS_STATUS_SUCCESS)
            return "hipBLASLt rejected the grouped problem";
        hipblaslt_ext::GemmPreference pref;
        pref.setMaxWorkspaceBytes(kWorkspace);
        std::vector<hipblasLtMatmulHeuristicResult_t> picks;
        (void)op_->algoGetHeuristic(1, pref, picks);
        if (picks.empty())
            return std::string("hipBLASLt has no grouped kernel for ") + dtype_name(p.dtype);
        std::vector<hipblaslt_ext::UserArguments> args(rows.size());
        lt_ok(op_->getDefaultValueForDeviceUserArguments(args.data()), "user arguments");
        const size_t bytes = args.size() * sizeof(hipblaslt_ext::UserArguments);
        hip_ok(hipMalloc(&device_args_, bytes), "argument buffer");
        hip_ok(hipMemcpyAsync(device_args_, args.data(), bytes, hipMemcpyHostToDevice, stream), "argument upload");
        lt_ok(op_->initialize(picks[0].algo, workspace_), "initialize");
        hip_ok(hipStreamSynchronize(stream), "prepare sync");
        kernel_ = op_->getKernelName();
        return "";
    }

    void run(hipStream_t stream) override { lt_ok(op_->run(device_args_, stream), "grouped run"); }

    void release() override {
        op_.reset();
        if (device_args_ != nullptr)
            (void)hipFree(device_args_);
        device_args_ = nullptr;
    }

    std::string detail() const override { return kernel_; }

private:
    hipblasLtHandle_t                           handle_      = nullptr;
    void                                       *workspace_   = nullptr;
    void                                       *device_args_ = nullptr;
    std::unique_ptr<hipblaslt_ext::GroupedGemm> op_;
    std::vector<float>                          scalars_; // alpha, beta per group (read by setProblem)
    std::string                                 kernel_;
};

} // namespace

std::unique_ptr<Backend> make_hipblaslt_loop_backend() { return std::make_unique<PerGroupLoop>(4); }
std::unique_ptr<Backend> make_hipblaslt_seq_backend() { return std::make_unique<PerGroupLoop>(1); }
std::unique_ptr<Backend> make_hipblaslt_grouped_backend() { return std::make_unique<LtGrouped>(); }

} // namespace tunemax

// Whether a kernel name is a stream-K solution's (the 4-stream gate's rule).
extern "C" int ggc_is_stream_k(const char *kernel_name) {
    return kernel_name != nullptr && tunemax::stream_k_kernel(kernel_name) ? 1 : 0;
}

// The heuristic's first choice for one group, by kernel name (no launch): what the 4-stream gate
// sees, for drivers and tests.
extern "C" int ggc_heuristic_kernel(int dtype, int64_t n, int64_t m, int64_t k, char *buf, size_t len) {
    try {
        hipblasLtHandle_t h = nullptr;
        tunemax::lt_ok(hipblasLtCreate(&h), "create handle");
        std::string name;
        try {
            const tunemax::GroupMatmul mm(dtype == 1 ? HIP_R_16F : HIP_R_16BF, n, m, k, tunemax::kLoopWorkspace);
            auto pick = mm.choose(h);
            name      = hipblaslt_ext::getKernelNameFromAlgo(h, pick.algo);
        } catch (...) {
            (void)hipblasLtDestroy(h);
            throw;
        }
        (void)hipblasLtDestroy(h);
        if (buf != nullptr && len > 0) {
            const size_t n_copy = name.size() < len - 1 ? name.size() : len - 1;
            name.copy(buf, n_copy);
            buf[n_copy] = '\0';
        }
        return tunemax::stream_k_kernel(name) ? 1 : 0;
    } catch (const std::exception &e) {
        if (buf != nullptr && len > 0) {
            const std::string msg = e.what();
            const size_t      n   = msg.size() < len - 1 ? msg.size() : len - 1;
            msg.copy(buf, n);
            buf[n] = '\0';
        }
        return -1;
    }
}
