// tunemax::Backend over the C ABI of the gfx950 kernel (include/gg_grouped_gemm.h).
// Takes the place of the reference's CkTileBackend (ck_kernel/ck_grouped_gemm.cpp:126-226):
// prepare -> gg_prepare (validate, device group table), run -> gg_run (one launch),
// release -> gg_release.
#include <stdexcept>
#include <string>

#include "backend.hpp"
#include "gg_grouped_gemm.h"

namespace tunemax {
namespace {

class Mi355xBackend final : public Backend {
public:
    ~Mi355xBackend() override { release(); }

    std::string name() const override { return "mi355x"; }

    std::string prepare(const GroupedGemmProblem &p, hipStream_t stream) override {
        release();
        if (static_cast<int64_t>(p.group_m.size()) != static_cast<int64_t>(p.group_num))
            throw std::runtime_error("group_m has " + std::to_string(p.group_m.size()) + " entries for " +
                                     std::to_string(p.group_num) + " groups");
        const int st = gg_prepare(p.dtype == DType::BF16 ? GG_DTYPE_BF16 : GG_DTYPE_FP16,
                                  p.group_num, p.n, p.k, p.group_m.data(), p.x, p.w, p.out,
                                  stream, &plan_);
        if (st == GG_ERR_UNSUPPORTED)
            return gg_last_error(); // reported as N/A
        if (st != GG_OK)
            throw std::runtime_error(std::string("gg_prepare: ") + gg_last_error());
        return "";
    }

    void run(hipStream_t stream) override {
        const int st = gg_run(plan_, stream);
        if (st != GG_OK)
            throw std::runtime_error(std::string("gg_run: ") + gg_last_error());
    }

    void release() override {
        gg_release(plan_);
        plan_ = nullptr;
    }

    std::string detail() const override { return plan_ ? gg_plan_detail(plan_) : ""; }

private:
    gg_plan *plan_ = nullptr;
};

} // namespace

std::unique_ptr<Backend> make_mi355x_backend() { return std::make_unique<Mi355xBackend>(); }

} // namespace tunemax
