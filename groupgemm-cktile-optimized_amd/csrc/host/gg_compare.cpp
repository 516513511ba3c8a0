// C shim over the comparison backends (gg_compare.h): exceptions become status codes and
// messages, so a Python driver sees an error instead of a terminated process.
#include <exception>
#include <memory>
#include <new>
#include <string>

#include "backend.hpp"
#include "gg_compare.h"

struct ggc_backend {
    std::unique_ptr<tunemax::Backend> impl;
    tunemax::GroupedGemmProblem       problem;
    std::string                       message, detail;
};

namespace {

int guarded(ggc_backend *b, int (*body)(ggc_backend *, void *), void *ctx) {
    if (b == nullptr)
        return 2;
    try {
        return body(b, ctx);
    } catch (const std::exception &e) {
        b->message = e.what();
    } catch (...) {
        b->message = "unknown exception";
    }
    return 2;
}

} // namespace

extern "C" {

int ggc_create(const char *name, ggc_backend **out) {
    if (out == nullptr || name == nullptr)
        return 2;
    *out = nullptr;
    const std::string n = name;
    try {
        std::unique_ptr<tunemax::Backend> impl;
        if (n == "hipblaslt_loop")
            impl = tunemax::make_hipblaslt_loop_backend();
        else if (n == "hipblaslt_seq")
            impl = tunemax::make_hipblaslt_seq_backend();
        else if (n == "hipblaslt_grouped")
            impl = tunemax::make_hipblaslt_grouped_backend();
        else
            return 1;
        *out         = new ggc_backend;
        (*out)->impl = std::move(impl);
        return 0;
    } catch (...) {
        return 2;
    }
}

struct PrepareArgs {
    int            dtype, group_num;
    int64_t        n, k;
    const int64_t *group_m, *lens;
    const void    *x, *w;
    void          *out, *stream;
};

int ggc_prepare(ggc_backend *b, int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                const int64_t *group_lens_pinned, const void *x, const void *w, void *out, void *stream) {
    PrepareArgs a{dtype, group_num, n, k, group_m, group_lens_pinned, x, w, out, stream};
    return guarded(
        b,
        [](ggc_backend *be, void *ctx) -> int {
            const PrepareArgs &q = *static_cast<PrepareArgs *>(ctx);
            be->message.clear();
            be->detail.clear();
            if (q.dtype != 0 && q.dtype != 1) {
                be->message = "dtype must be 0 (bf16) or 1 (fp16)";
                return 2;
            }
            if (q.group_num < 0 || (q.group_num > 0 && q.group_m == nullptr)) {
                be->message = "group sizes missing";
                return 2;
            }
            tunemax::GroupedGemmProblem &p = be->problem;
            p.dtype                        = q.dtype == 0 ? tunemax::DType::BF16 : tunemax::DType::FP16;
            p.group_num                    = q.group_num;
            p.n                            = q.n;
            p.k                            = q.k;
            p.group_m.assign(q.group_m, q.group_m + q.group_num);
            p.x                 = q.x;
            p.w                 = q.w;
            p.out               = q.out;
            p.group_lens_pinned = q.lens;
            const std::string why = be->impl->prepare(p, static_cast<hipStream_t>(q.stream));
            if (!why.empty()) {
                be->message = why;
                return 1;
            }
            be->detail = be->impl->detail();
            return 0;
        },
        &a);
}

int ggc_run(ggc_backend *b, void *stream) {
    return guarded(
        b,
        [](ggc_backend *be, void *ctx) -> int {
            be->impl->run(static_cast<hipStream_t>(ctx));
            return 0;
        },
        stream);
}

void ggc_release(ggc_backend *b) {
    if (b != nullptr)
        (void)guarded(
            b,
            [](ggc_backend *be, void *) -> int {
                be->impl->release();
                return 0;
            },
            nullptr);
}

void ggc_destroy(ggc_backend *b) {
    if (b == nullptr)
        return;
    try {
        delete b;
    } catch (...) {
    }
}

const char *ggc_message(const ggc_backend *b) { return b != nullptr ? b->message.c_str() : ""; }

const char *ggc_detail(const ggc_backend *b) { return b != nullptr ? b->detail.c_str() : ""; }

} // extern "C"
