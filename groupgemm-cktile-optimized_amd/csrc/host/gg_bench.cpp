// gg_bench: grouped-GEMM backends over a shape list, one CSV row per (case, backend).
//
//   gg_bench --shapes shapes/configs.csv [--dtype bf16|fp16] [--backends mi355x,hipblaslt_seq]
//            [--only 1001,1005] [--warmup 20] [--iters 100] [--no-check] [--out rows.csv] [--verbose]
//            [--clock]
//
// What it keeps of the reference's driver (bench/bench_main.cpp), so that its CSVs compare row
// for row with the reference's: the flags (:8-10), the CSV header (:306), balanced groups of M
// rows with x and w ~ N(0,1) from seeds 1 and 2 (:436, 451-456, through gg_fill_randn), the
// output zeroed before each backend (:467-468), prepare() untimed, one run() checked at 4
// corners + 256 random positions per group drawn from one mt19937_64(1234) (row, then column;
// :210-227) with |got - ref| <= 1e-2 + 1e-2 |ref| and NaN a mismatch (:264-268), then
// `warmup` runs and `iters` runs between two HIP events (:490-501), and exit status 1 when a row
// FAILs or ERRORs (:534-536).
//
// How it does it is its own:
//   * backends come from tunemax::backend_registry() by name;
//   * one device arena, sized up front for the largest selected case, holds x, w and out for
//     every case (no free / malloc between cases), with the pinned group lengths beside it;
//   * the check is one launch with a wave per sampled output (fp32 dot over K, lane-strided,
//     reduced with cross-lane adds), buffers allocated once for the largest case;
//   * the summary compares every backend with the first one: geomean speedup and wins over the
//     cases every backend passed;
//   * --clock runs gg_clock_probe (one wave reading the shader clock against the wall clock) on a
//     second stream over the first 60 % of the mi355x backend's timed loop and appends the
//     effective clock to the row's Detail ("[clock 1712 MHz]"). Only there: the probe's wave needs a
//     CU slot beside the GEMM's workgroups, which the mi355x kernel leaves (a few VGPRs, no LDS),
//     while hipBLASLt's kernels can fill a CU's registers, so that the probe displaces one of their
//     workgroups and both the timing and the clock it reads are no longer the kernel's own.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <ctime>
#include <exception>
#include <fstream>
#include <functional>
#include <iostream>
#include <map>
#include <random>
#include <set>
#include <sstream>
#include <string>
#include <string_view>
#include <vector>

#include "backend.hpp"
#include "gg_grouped_gemm.h"

namespace ggb {

using tunemax::Backend;
using tunemax::DType;
using tunemax::GroupedGemmProblem;

[[noreturn]] void die(const std::string &why, int code = 2) {
    std::fprintf(stderr, "gg_bench: %s\n", why.c_str());
    std::exit(code);
}

void hip_or_die(hipError_t e, const char *what) {
    if (e != hipSuccess)
        die(std::string(what) + ": " + hipGetErrorString(e), 1);
}

// Fields of one comma-separated line, trimmed of blanks and carriage returns.
std::vector<std::string> fields(std::string_view line) {
    std::vector<std::string> out;
    while (true) {
        const size_t     cut = line.find(',');
        std::string_view f   = line.substr(0, cut);
        while (!f.empty() && (f.front() == ' ' || f.front() == '\t'))
            f.remove_prefix(1);
        while (!f.empty() && (f.back() == ' ' || f.back() == '\t' || f.back() == '\r'))
            f.remove_suffix(1);
        out.emplace_back(f);
        if (cut == std::string_view::npos)
            break;
        line.remove_prefix(cut + 1);
    }
    return out;
}

// ---- settings: a table of flags ------------------------------------------------------------
struct Settings {
    std::string              shapes, out;
    DType                    dtype = DType::BF16;
    std::vector<std::string> backends{"mi355x", "hipblaslt_grouped", "hipblaslt_loop"};
    std::set<int>            only;
    int                      warmup = 20, iters = 100;
    bool                     check = true, verbose = false, clock = false;
};

const char *kUsage = "usage: gg_bench --shapes FILE.csv [--dtype bf16|fp16] [--backends a,b,...] [--only ID,...]\n"
                     "                [--warmup N] [--iters N] [--no-check] [--out FILE.csv] [--verbose] [--clock]\n";

Settings parse(int argc, char **argv) {
    Settings s;
    auto     ints = [](const std::string &v) {
        std::vector<int> r;
        for (const auto &f : fields(v))
            if (!f.empty())
                r.push_back(std::stoi(f));
        return r;
    };
    struct Flag {
        const char                              *name;
        bool                                     takes_value;
        std::function<void(const std::string &)> apply;
    };
    const Flag table[] = {
        {"--shapes", true, [&](const std::string &v) { s.shapes = v; }},
        {"--out", true, [&](const std::string &v) { s.out = v; }},
        {"--dtype", true,
         [&](const std::string &v) {
             if (v != "bf16" && v != "fp16")
                 die("--dtype takes bf16 or fp16\n" + std::string(kUsage));
             s.dtype = v == "bf16" ? DType::BF16 : DType::FP16;
         }},
        {"--backends", true,
         [&](const std::string &v) {
             s.backends.clear();
             for (const auto &f : fields(v))
                 if (!f.empty())
                     s.backends.push_back(f);
         }},
        {"--only", true,
         [&](const std::string &v) {
             for (int id : ints(v))
                 s.only.insert(id);
         }},
        {"--warmup", true, [&](const std::string &v) { s.warmup = std::stoi(v); }},
        {"--iters", true, [&](const std::string &v) { s.iters = std::stoi(v); }},
        {"--no-check", false, [&](const std::string &) { s.check = false; }},
        {"--verbose", false, [&](const std::string &) { s.verbose = true; }},
        {"--clock", false, [&](const std::string &) { s.clock = true; }},
    };
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        if (arg == "-h" || arg == "--help") {
            std::fputs(kUsage, stdout);
            std::exit(0);
        }
        const Flag *f = nullptr;
        for (const auto &cand : table)
            if (arg == cand.name)
                f = &cand;
        if (f == nullptr)
            die("unknown argument " + arg + "\n" + kUsage);
        if (f->takes_value && i + 1 >= argc)
            die(arg + " needs a value\n" + kUsage);
        try {
            f->apply(f->takes_value ? std::string(argv[++i]) : std::string());
        } catch (const std::exception &) {
            die("bad value for " + arg + "\n" + kUsage);
        }
    }
    if (s.shapes.empty())
        die("--shapes is required\n" + std::string(kUsage));
    if (s.iters < 1 || s.warmup < 0)
        die("--iters must be at least 1 and --warmup at least 0");
    if (s.backends.empty())
        die("--backends names no backend");
    return s;
}

// ---- the shape list: TestID, Case, B, M, N, K, columns found by name -----------------------------
struct Shape {
    int         id = 0;
    std::string label;
    int64_t     b = 0, m = 0, n = 0, k = 0;
    size_t      x_elems() const { return size_t(b * m * k); }
    size_t      w_elems() const { return size_t(b * n * k); }
    size_t      out_elems() const { return size_t(b * m * n); }
};

std::vector<Shape> load_shapes(const std::string &path, const std::set<int> &only) {
    std::ifstream in(path);
    if (!in)
        die("cannot read " + path);
    std::string line;
    if (!std::getline(in, line))
        die(path + " is empty");
    const auto              head = fields(line);
    std::map<std::string, size_t> at;
    for (size_t i = 0; i < head.size(); ++i)
        at[head[i]] = i;
    for (const char *col : {"TestID", "Case", "B", "M", "N", "K"})
        if (at.count(col) == 0)
            die(path + " has no column " + col);
    std::vector<Shape> shapes;
    int                line_no = 1;
    while (std::getline(in, line)) {
        ++line_no;
        if (line.find_first_not_of(" \t\r") == std::string::npos)
            continue;
        const auto v = fields(line);
        if (v.size() < head.size())
            die(path + ":" + std::to_string(line_no) + ": too few fields");
        Shape s;
        try {
            s.id    = std::stoi(v[at["TestID"]]);
            s.label = v[at["Case"]];
            s.b     = std::stoll(v[at["B"]]);
            s.m     = std::stoll(v[at["M"]]);
            s.n     = std::stoll(v[at["N"]]);
            s.k     = std::stoll(v[at["K"]]);
        } catch (const std::exception &) {
            die(path + ":" + std::to_string(line_no) + ": not a number");
        }
        if (s.b < 0 || s.m < 0 || s.n < 0 || s.k < 0)
            die(path + ":" + std::to_string(line_no) + ": negative size");
        if (only.empty() || only.count(s.id) != 0)
            shapes.push_back(s);
    }
    return shapes;
}

// ---- device memory: one arena for the whole run ------------------------------------------------
// x, w and out of every case live in one allocation sized for the largest selected case (each
// part 256-byte aligned); the group lengths sit in pinned host memory beside it (the per-group
// hipBLASLt loops read them on the host every run).
class Arena {
public:
    explicit Arena(const std::vector<Shape> &shapes) {
        for (const auto &s : shapes) {
            x_max_   = std::max(x_max_, round_up(s.x_elems() * 2));
            w_max_   = std::max(w_max_, round_up(s.w_elems() * 2));
            out_max_ = std::max(out_max_, round_up(s.out_elems() * 2));
            groups_  = std::max(groups_, size_t(s.b));
        }
        hip_or_die(hipMalloc(&base_, std::max<size_t>(x_max_ + w_max_ + out_max_, 256)), "device arena");
        hip_or_die(hipHostMalloc(reinterpret_cast<void **>(&lens_), std::max<size_t>(groups_, 1) * sizeof(int64_t)),
                   "pinned group lengths");
    }
    Arena(const Arena &)            = delete;
    Arena &operator=(const Arena &) = delete;
    ~Arena() {
        (void)hipFree(base_);
        (void)hipHostFree(lens_);
    }

    // The problem of shape s (balanced groups) on the arena's memory.
    GroupedGemmProblem problem(const Shape &s, DType t) const {
        GroupedGemmProblem p;
        p.dtype     = t;
        p.group_num = int(s.b);
        p.n         = s.n;
        p.k         = s.k;
        p.group_m.assign(size_t(s.b), s.m);
        std::fill(lens_, lens_ + s.b, s.m);
        p.group_lens_pinned = lens_;
        p.x                 = base_;
        p.w                 = static_cast<char *>(base_) + x_max_;
        p.out               = static_cast<char *>(base_) + x_max_ + w_max_;
        return p;
    }
    size_t bytes() const { return x_max_ + w_max_ + out_max_; }

private:
    static size_t round_up(size_t b) { return (b + 255) / 256 * 256; }
    void         *base_ = nullptr;
    int64_t      *lens_ = nullptr;
    size_t        x_max_ = 0, w_max_ = 0, out_max_ = 0, groups_ = 0;
};

// ---- the sampled check -----------------------------------------------------------------------
struct Probe {
    int64_t row, col, group; // output row (global), output column, its group
};

// Per group with rows: its four corners, then 256 (row, column) draws from one mt19937_64(1234)
// shared by all groups, the row drawn first.
std::vector<Probe> probes_for(const GroupedGemmProblem &p) {
    std::mt19937_64    rng(1234);
    std::vector<Probe> probes;
    int64_t            first = 0;
    for (int g = 0; g < p.group_num; ++g) {
        const int64_t m = p.group_m[size_t(g)];
        if (m > 0 && p.n > 0) {
            const int64_t last = first + m - 1;
            for (const int64_t r : {first, last})
                for (const int64_t c : {int64_t(0), p.n - 1})
                    probes.push_back({r, c, g});
            for (int i = 0; i < 256; ++i) {
                const int64_t r = first + int64_t(rng() % uint64_t(m));
                const int64_t c = int64_t(rng() % uint64_t(p.n));
                probes.push_back({r, c, g});
            }
        }
        first += m;
    }
    return probes;
}

__device__ inline float as_float(uint16_t v, bool fp16) {
    return fp16 ? static_cast<float>(__builtin_bit_cast(_Float16, v)) : __uint_as_float(uint32_t(v) << 16);
}

// One wave per probe: lanes take every 64th K element of x[row] . w[group][col] in fp32, the
// partial sums meet through cross-lane adds; lane 0 writes the reference and the stored output.
__global__ void __launch_bounds__(256)
probe_kernel(const uint16_t *x, const uint16_t *w, const uint16_t *out, int64_t n, int64_t k, int fp16,
             const Probe *probes, int count, float *ref, float *got) {
    const int pi   = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    const int lane = int(threadIdx.x & 63);
    if (pi >= count)
        return;
    const Probe     pr = probes[pi];
    const uint16_t *xr = x + pr.row * k;
    const uint16_t *wr = w + (pr.group * n + pr.col) * k;
    float           s  = 0.0f;
    for (int64_t i = lane; i < k; i += 64)
        s += as_float(xr[i], fp16 != 0) * as_float(wr[i], fp16 != 0);
    for (int d = 32; d >= 1; d >>= 1)
        s += __shfl_xor(s, d, 64);
    if (lane == 0) {
        ref[pi] = s;
        got[pi] = as_float(out[pr.row * n + pr.col], fp16 != 0);
    }
}

struct Verdict {
    int    off     = 0;   // outputs outside the tolerance (NaN included)
    double max_abs = 0.0; // infinite when an output is NaN
};

class Checker {
public:
    explicit Checker(size_t max_probes) : cap_(std::max<size_t>(max_probes, 1)) {
        hip_or_die(hipMalloc(&probes_, cap_ * sizeof(Probe)), "probe buffer");
        hip_or_die(hipMalloc(&vals_, 2 * cap_ * sizeof(float)), "probe values");
    }
    Checker(const Checker &)            = delete;
    Checker &operator=(const Checker &) = delete;
    ~Checker() {
        (void)hipFree(probes_);
        (void)hipFree(vals_);
    }

    Verdict verify(const GroupedGemmProblem &p, const std::vector<Probe> &probes, hipStream_t s) {
        Verdict v;
        if (probes.empty())
            return v;
        const int count = int(probes.size());
        hip_or_die(hipMemcpyAsync(probes_, probes.data(), probes.size() * sizeof(Probe), hipMemcpyHostToDevice, s),
                   "probe upload");
        hipLaunchKernelGGL(probe_kernel, dim3(unsigned((count + 3) / 4)), dim3(256), 0, s,
                           static_cast<const uint16_t *>(p.x), static_cast<const uint16_t *>(p.w),
                           static_cast<const uint16_t *>(p.out), p.n, p.k, p.dtype == DType::FP16 ? 1 : 0,
                           probes_, count, vals_, vals_ + cap_);
        hip_or_die(hipGetLastError(), "probe launch");
        std::vector<float> ref(probes.size()), got(probes.size());
        hip_or_die(hipMemcpyAsync(ref.data(), vals_, ref.size() * sizeof(float), hipMemcpyDeviceToHost, s), "ref");
        hip_or_die(hipMemcpyAsync(got.data(), vals_ + cap_, got.size() * sizeof(float), hipMemcpyDeviceToHost, s),
                   "got");
        hip_or_die(hipStreamSynchronize(s), "check sync");
        for (size_t i = 0; i < ref.size(); ++i) {
            const double e = std::fabs(double(got[i]) - double(ref[i]));
            v.max_abs      = std::max(v.max_abs, std::isnan(e) ? INFINITY : e);
            v.off += !(e <= 1e-2 + 1e-2 * std::fabs(double(ref[i])));
        }
        return v;
    }

private:
    size_t cap_;
    Probe *probes_ = nullptr;
    float *vals_   = nullptr; // ref [cap_], then got [cap_]
};

// ---- the report: CSV rows, console lines, summary ----------------------------------------------
struct Result {
    const Shape *shape = nullptr;
    std::string  backend, check, detail;
    double       ms = NAN, tflops = NAN, max_abs = NAN;
};

std::string quoted(const std::string &s) {
    std::string q = "\"";
    for (const char c : s)
        q += c == '"' ? std::string("\"\"") : std::string(1, c);
    return q + "\"";
}

std::string fixed(double v, int digits) {
    char buf[64];
    std::snprintf(buf, sizeof(buf), "%.*f", digits, v);
    return buf;
}

class Report {
public:
    Report(std::string path, std::string gpu, DType t) : path_(std::move(path)), gpu_(std::move(gpu)), dtype_(t) {}

    void add(Result r) {
        std::printf("  %-18s %-6s %12s %12s  %.100s\n", r.backend.c_str(), r.check.c_str(),
                    std::isnan(r.ms) ? "-" : (fixed(r.ms, 4) + " ms").c_str(),
                    std::isnan(r.tflops) ? "-" : (fixed(r.tflops, 1) + " TF").c_str(), r.detail.c_str());
        std::fflush(stdout);
        results_.push_back(std::move(r));
    }

    // The whole table so far (rewritten after every case, so an interrupted run keeps what ran).
    void write() const {
        std::ofstream f(path_);
        if (!f)
            die("cannot write " + path_, 1);
        f << "TestID,Case,B,M,N,K,Dtype,GPU,Backend,Check,Time_ms,TFLOPS,MaxAbsErr,Detail\n";
        for (const auto &r : results_) {
            const Shape &s = *r.shape;
            f << s.id << ',' << s.label << ',' << s.b << ',' << s.m << ',' << s.n << ',' << s.k << ','
              << tunemax::dtype_name(dtype_) << ',' << quoted(gpu_) << ',' << r.backend << ',' << r.check << ','
              << (std::isnan(r.ms) ? std::string(",") : fixed(r.ms, 4) + "," + fixed(r.tflops, 2)) << ','
              << (std::isnan(r.max_abs) ? std::string() : fixed(r.max_abs, 4)) << ',' << quoted(r.detail) << '\n';
        }
    }

    // Every backend against the first one, over the cases that all backends passed.
    void summary(const std::vector<std::string> &names) const {
        std::map<int, std::map<std::string, const Result *>> by_case;
        for (const auto &r : results_)
            by_case[r.shape->id][r.backend] = &r;
        std::vector<int> common;
        for (const auto &[id, rows] : by_case) {
            bool ok = rows.size() == names.size();
            for (const auto &[name, r] : rows)
                ok = ok && r->check == "PASS";
            if (ok)
                common.push_back(id);
        }
        std::printf("\nsummary: %zu of %zu cases passed on every backend\n", common.size(), by_case.size());
        if (common.empty())
            return;
        const std::string &base = names.front();
        std::printf("  %-18s %12s %12s %22s\n", "backend", "mean TFLOPS", "total ms",
                    (base + " speedup (wins)").c_str());
        for (const auto &name : names) {
            double tf = 0.0, ms = 0.0, log_speedup = 0.0;
            int    wins = 0;
            for (const int id : common) {
                const Result *r = by_case[id][name], *b = by_case[id][base];
                tf += r->tflops;
                ms += r->ms;
                log_speedup += std::log(r->ms / b->ms);
                wins += b->ms < r->ms;
            }
            std::printf("  %-18s %12.1f %12.3f %14.3fx (%d/%zu)\n", name.c_str(), tf / double(common.size()), ms,
                        std::exp(log_speedup / double(common.size())), wins, common.size());
        }
        std::printf("  (speedup = backend time / %s time, geometric mean; wins = cases %s was faster)\n",
                    base.c_str(), base.c_str());
    }

    bool failed() const {
        return std::any_of(results_.begin(), results_.end(),
                           [](const Result &r) { return r.check == "FAIL" || r.check == "ERROR"; });
    }
    const std::string &path() const { return path_; }

private:
    std::string         path_, gpu_;
    DType               dtype_;
    std::vector<Result> results_;
};

std::string default_path(const Settings &s) {
    std::string stem = s.shapes.substr(s.shapes.find_last_of('/') + 1);
    stem             = stem.substr(0, stem.find('.'));
    char              stamp[32];
    const std::time_t now = std::time(nullptr);
    std::strftime(stamp, sizeof(stamp), "%Y%m%d-%H%M%S", std::localtime(&now));
    return "results/" + stem + "_" + tunemax::dtype_name(s.dtype) + "_" + stamp + ".csv";
}

// ---- one backend on one case -----------------------------------------------------------------
struct Clock {
    hipEvent_t  a = nullptr, b = nullptr, w = nullptr; // w: start of the warmup (--clock)
    hipStream_t side  = nullptr;                       // the clock probe's stream (default priority)
    uint64_t   *words = nullptr;                       // its five result words (device)
    Clock() {
        hip_or_die(hipEventCreate(&a), "event");
        hip_or_die(hipEventCreate(&b), "event");
        hip_or_die(hipEventCreate(&w), "event");
        hip_or_die(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "probe stream");
        hip_or_die(hipMalloc(&words, 5 * sizeof(uint64_t)), "probe words");
    }
    ~Clock() {
        (void)hipFree(words);
        (void)hipStreamDestroy(side);
        (void)hipEventDestroy(w);
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
};

Result run_backend(Backend &be, const Shape &shape, const GroupedGemmProblem &p, const std::vector<Probe> &probes,
                   const Settings &set, Checker &checker, Clock &clock, hipStream_t s) {
    Result r;
    r.shape   = &shape;
    r.backend = be.name();
    auto note = [&](const char *phase) {
        if (set.verbose)
            std::fprintf(stderr, "[gg_bench %ld] %s %s\n", long(std::time(nullptr)), r.backend.c_str(), phase);
    };
    try {
        hip_or_die(hipMemsetAsync(p.out, 0, size_t(p.total_m()) * size_t(p.n) * 2, s), "output clear");
        note("prepare");
        const std::string why = be.prepare(p, s);
        if (!why.empty()) {
            r.check  = "N/A";
            r.detail = why;
            be.release();
            return r;
        }
        r.detail = be.detail();
        note("first run");
        be.run(s);
        hip_or_die(hipStreamSynchronize(s), "first run");
        if (set.check) {
            const Verdict v = checker.verify(p, probes, s);
            r.check         = v.off == 0 ? "PASS" : "FAIL";
            r.max_abs       = v.max_abs;
            if (v.off != 0)
                r.detail += " | " + std::to_string(v.off) + "/" + std::to_string(probes.size()) + " samples off";
        } else {
            r.check = "SKIP";
        }
        note("timing");
        hip_or_die(hipEventRecord(clock.w, s), "warmup event");
        for (int i = 0; i < set.warmup; ++i)
            be.run(s);
        hip_or_die(hipEventRecord(clock.a, s), "start event");
        const bool probe = set.clock && r.backend == "mi355x";
        if (probe) {
            // the probe starts with the timed loop and spans 60 % of it (its length estimated
            // from the warmup)
            hip_or_die(hipEventSynchronize(clock.a), "warmup sync");
            float warm = 0.0f;
            hip_or_die(hipEventElapsedTime(&warm, clock.w, clock.a), "warmup time");
            const double per = set.warmup > 0 ? double(warm) / set.warmup : 1.0;
            hip_or_die(hipStreamWaitEvent(clock.side, clock.a, 0), "probe wait");
            if (gg_clock_probe(clock.words, 0.6e-3 * per * set.iters, clock.side) != GG_OK)
                throw std::runtime_error(std::string("clock probe: ") + gg_last_error());
        }
        for (int i = 0; i < set.iters; ++i)
            be.run(s);
        hip_or_die(hipEventRecord(clock.b, s), "stop event");
        hip_or_die(hipEventSynchronize(clock.b), "stop sync");
        float total = 0.0f;
        hip_or_die(hipEventElapsedTime(&total, clock.a, clock.b), "elapsed");
        r.ms     = double(total) / set.iters;
        r.tflops = p.flops() / (r.ms * 1e-3) / 1e12;
        if (probe) {
            uint64_t v[5] = {};
            hip_or_die(hipStreamSynchronize(clock.side), "probe sync");
            hip_or_die(hipMemcpy(v, clock.words, sizeof(v), hipMemcpyDeviceToHost), "probe words");
            if (v[3] > v[1] && v[4] > 0)
                r.detail += " [clock " + std::to_string(std::llround(double(v[2] - v[0]) / (double(v[3] - v[1]) / double(v[4])) / 1e6)) + " MHz]";
        }
    } catch (const std::exception &e) {
        (void)hipStreamSynchronize(s);
        r.check  = "ERROR";
        r.detail = e.what();
    }
    be.release();
    note("done");
    return r;
}

int main_(int argc, char **argv) {
    const Settings set = parse(argc, argv);
    std::vector<std::unique_ptr<Backend>> backends;
    for (const auto &name : set.backends) {
        const auto &reg = tunemax::backend_registry();
        const auto  it  = reg.find(name);
        if (it == reg.end()) {
            std::string known;
            for (const auto &[k, f] : reg)
                known += " " + k;
            die("unknown backend " + name + " (known:" + known + ")");
        }
        backends.push_back(it->second());
    }
    const std::vector<Shape> shapes = load_shapes(set.shapes, set.only);

    hipDeviceProp_t prop;
    hip_or_die(hipGetDeviceProperties(&prop, 0), "device properties");
    const std::string gpu = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    Arena             arena(shapes);
    size_t            most_probes = 0;
    for (const auto &sh : shapes)
        most_probes = std::max(most_probes, size_t(sh.b) * 260);
    Checker     checker(most_probes);
    Clock       clock;
    hipStream_t s = nullptr;
    hip_or_die(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream");
    Report report(set.out.empty() ? default_path(set) : set.out, gpu, set.dtype);

    std::printf("%s: %zu cases from %s, %s, warmup %d, iters %d, arena %.1f GB\n", gpu.c_str(), shapes.size(),
                set.shapes.c_str(), tunemax::dtype_name(set.dtype), set.warmup, set.iters, double(arena.bytes()) / 1e9);
    for (const auto &shape : shapes) {
        const GroupedGemmProblem p = arena.problem(shape, set.dtype);
        const int                d = set.dtype == DType::BF16 ? GG_DTYPE_BF16 : GG_DTYPE_FP16;
        if (gg_fill_randn(d, const_cast<void *>(p.x), shape.x_elems(), 1, s) != GG_OK ||
            gg_fill_randn(d, const_cast<void *>(p.w), shape.w_elems(), 2, s) != GG_OK)
            die(std::string("input fill: ") + gg_last_error(), 1);
        const std::vector<Probe> probes = set.check ? probes_for(p) : std::vector<Probe>{};
        std::printf("\n[%d] %s  %ld x %ld, N %ld, K %ld  (%.3f TFLOP)\n", shape.id, shape.label.c_str(), long(shape.b),
                    long(shape.m), long(shape.n), long(shape.k), p.flops() / 1e12);
        for (auto &be : backends)
            report.add(run_backend(*be, shape, p, probes, set, checker, clock, s));
        report.write();
    }
    report.summary(set.backends);
    std::printf("\nresults: %s\n", report.path().c_str());
    (void)hipStreamDestroy(s);
    return report.failed() ? 1 : 0;
}

} // namespace ggb

int main(int argc, char **argv) { return ggb::main_(argc, argv); }
