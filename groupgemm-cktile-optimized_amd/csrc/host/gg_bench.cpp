// Grouped-GEMM benchmark driver: same command line, input generation, correctness check,
// timing protocol, result CSV and summary as the reference's tunemax_bench
// (bench/bench_main.cpp:8-10, 71-113, 124-149, 160-272, 316-381, 392-538), with backends
// looked up by name in tunemax::backend_registry().
//
//   gg_bench --shapes shapes/configs.csv [--dtype bf16|fp16] [--backends a,b,c]
//            [--only 1,2] [--warmup 20] [--iters 100] [--no-check] [--out results.csv] [--verbose]
//
// Per case: B balanced groups of M rows, x and w ~ N(0,1) (seeds 1 and 2), output zeroed
// before each backend, prepare() untimed, one run() + sampled fp32 check (4 corners and 256
// random outputs per group from mt19937_64(1234), |got - ref| <= 1e-2 + 1e-2 |ref|), then
// warmup and `iters` back-to-back run() calls between two HIP events -> mean ms, TFLOPS.
// Exit status 1 if any row is FAIL or ERROR.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <ctime>
#include <exception>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <map>
#include <random>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "backend.hpp"
#include "gg_grouped_gemm.h"

namespace tunemax {
namespace {

struct Options {
    std::string              shapes, out;
    DType                    dtype = DType::BF16;
    std::vector<std::string> backends{"mi355x", "hipblaslt_loop", "hipblaslt_grouped"};
    std::set<int>            only;
    int                      warmup = 20, iters = 100;
    bool                     check = true;
    bool                     verbose = false; // phase timestamps per backend on stderr
};

std::vector<std::string> split(const std::string &s, char sep) {
    std::vector<std::string> parts;
    std::stringstream        ss(s);
    std::string              item;
    while (std::getline(ss, item, sep)) {
        while (!item.empty() && (item.back() == '\r' || item.back() == ' '))
            item.pop_back();
        while (!item.empty() && item.front() == ' ')
            item.erase(item.begin());
        if (!item.empty())
            parts.push_back(item);
    }
    return parts;
}

[[noreturn]] void usage(const std::string &msg) {
    std::cerr << "error: " << msg << "\n"
              << "usage: gg_bench --shapes FILE.csv [--dtype bf16|fp16] [--backends a,b,...]\n"
              << "                [--only TESTID,...] [--warmup N] [--iters N] [--no-check] [--out FILE.csv]\n"
              << "                [--verbose]   (phase timestamps per backend on stderr)\n"
              << "backends:";
    for (const auto &kv : backend_registry())
        std::cerr << " " << kv.first;
    std::cerr << "\n";
    std::exit(2);
}

Options parse_args(int argc, char **argv) {
    Options o;
    for (int i = 1; i < argc; ++i) {
        const std::string a    = argv[i];
        auto              next = [&]() -> std::string {
            if (i + 1 >= argc)
                usage("missing value for " + a);
            return argv[++i];
        };
        if (a == "--shapes")
            o.shapes = next();
        else if (a == "--out")
            o.out = next();
        else if (a == "--dtype") {
            const std::string d = next();
            if (d != "bf16" && d != "fp16")
                usage("--dtype must be bf16 or fp16");
            o.dtype = d == "bf16" ? DType::BF16 : DType::FP16;
        } else if (a == "--backends")
            o.backends = split(next(), ',');
        else if (a == "--only")
            for (const auto &id : split(next(), ','))
                o.only.insert(std::stoi(id));
        else if (a == "--warmup")
            o.warmup = std::stoi(next());
        else if (a == "--iters")
            o.iters = std::stoi(next());
        else if (a == "--no-check")
            o.check = false;
        else if (a == "--verbose")
            o.verbose = true;
        else if (a == "-h" || a == "--help")
            usage("help requested");
        else
            usage("unknown argument " + a);
    }
    if (o.shapes.empty())
        usage("--shapes is required");
    if (o.iters < 1 || o.warmup < 0)
        usage("--iters must be >= 1 and --warmup >= 0");
    for (const auto &b : o.backends)
        if (!backend_registry().count(b))
            usage("unknown backend " + b);
    return o;
}

struct Case {
    int         id;
    std::string name;
    int64_t     b, m, n, k;
};

std::vector<Case> read_cases(const std::string &path) {
    std::ifstream f(path);
    if (!f)
        usage("cannot open " + path);
    std::string header;
    std::getline(f, header);
    std::map<std::string, size_t> col;
    const auto                    names = split(header, ',');
    for (size_t i = 0; i < names.size(); ++i)
        col[names[i]] = i;
    for (const char *need : {"TestID", "Case", "B", "M", "N", "K"})
        if (!col.count(need))
            usage(path + ": missing column " + need);
    std::vector<Case> cases;
    std::string       line;
    while (std::getline(f, line)) {
        const auto v = split(line, ',');
        if (v.size() < names.size())
            continue;
        cases.push_back({std::stoi(v[col["TestID"]]), v[col["Case"]], std::stoll(v[col["B"]]),
                         std::stoll(v[col["M"]]), std::stoll(v[col["N"]]), std::stoll(v[col["K"]])});
    }
    return cases;
}

// ---- sampled fp32 reference on the device --------------------------------------------------
struct Sample {
    int64_t row, col, group;
};

__device__ float to_f32(uint16_t h, bool fp16) {
    return fp16 ? static_cast<float>(__builtin_bit_cast(_Float16, h))
                : __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// One block per sample: fp32 dot of x[row, :] and w[group][col, :], plus the backend's value.
__global__ void sampled_reference(const uint16_t *x, const uint16_t *w, const uint16_t *out, int64_t n,
                                  int64_t k, bool fp16, const Sample *samples, float *ref, float *got) {
    const Sample    s  = samples[blockIdx.x];
    const uint16_t *xr = x + s.row * k;
    const uint16_t *wr = w + (s.group * n + s.col) * k;
    float           acc = 0.f;
    for (int64_t i = threadIdx.x; i < k; i += blockDim.x)
        acc += to_f32(xr[i], fp16) * to_f32(wr[i], fp16);
    __shared__ float part[256];
    part[threadIdx.x] = acc;
    __syncthreads();
    for (unsigned half = blockDim.x / 2; half > 0; half /= 2) {
        if (threadIdx.x < half)
            part[threadIdx.x] += part[threadIdx.x + half];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        ref[blockIdx.x] = part[0];
        got[blockIdx.x] = to_f32(out[s.row * n + s.col], fp16);
    }
}

std::vector<Sample> make_samples(const GroupedGemmProblem &p) {
    std::mt19937_64     rng(1234);
    std::vector<Sample> s;
    int64_t             row0 = 0;
    for (int g = 0; g < p.group_num; ++g) {
        const int64_t m = p.group_m[g];
        if (m > 0) {
            for (const int64_t r : {row0, row0 + m - 1})
                for (const int64_t c : {int64_t(0), p.n - 1})
                    s.push_back({r, c, g});
            for (int i = 0; i < 256; ++i) {
                const int64_t r = row0 + int64_t(rng() % uint64_t(m)); // row drawn first
                const int64_t c = int64_t(rng() % uint64_t(p.n));
                s.push_back({r, c, g});
            }
        }
        row0 += m;
    }
    return s;
}

struct CheckResult {
    bool   pass       = false;
    double max_abs    = 0;
    int    mismatches = 0;
};

CheckResult check_output(const GroupedGemmProblem &p, const std::vector<Sample> &samples, hipStream_t stream) {
    const size_t ns = samples.size();
    Sample      *d_s;
    float       *d_ref, *d_got;
    TUNEMAX_HIP_CHECK(hipMalloc(&d_s, ns * sizeof(Sample)));
    TUNEMAX_HIP_CHECK(hipMalloc(&d_ref, ns * sizeof(float)));
    TUNEMAX_HIP_CHECK(hipMalloc(&d_got, ns * sizeof(float)));
    TUNEMAX_HIP_CHECK(hipMemcpyAsync(d_s, samples.data(), ns * sizeof(Sample), hipMemcpyHostToDevice, stream));
    hipLaunchKernelGGL(sampled_reference, dim3(ns), dim3(256), 0, stream, static_cast<const uint16_t *>(p.x),
                       static_cast<const uint16_t *>(p.w), static_cast<const uint16_t *>(p.out), p.n, p.k,
                       p.dtype == DType::FP16, d_s, d_ref, d_got);
    TUNEMAX_HIP_CHECK(hipGetLastError());
    std::vector<float> ref(ns), got(ns);
    TUNEMAX_HIP_CHECK(hipMemcpyAsync(ref.data(), d_ref, ns * sizeof(float), hipMemcpyDeviceToHost, stream));
    TUNEMAX_HIP_CHECK(hipMemcpyAsync(got.data(), d_got, ns * sizeof(float), hipMemcpyDeviceToHost, stream));
    TUNEMAX_HIP_CHECK(hipStreamSynchronize(stream));
    TUNEMAX_HIP_CHECK(hipFree(d_s));
    TUNEMAX_HIP_CHECK(hipFree(d_ref));
    TUNEMAX_HIP_CHECK(hipFree(d_got));
    CheckResult r;
    for (size_t i = 0; i < ns; ++i) {
        const double err = std::fabs(double(got[i]) - double(ref[i]));
        r.max_abs        = std::max(r.max_abs, std::isnan(err) ? INFINITY : err);
        if (!(err <= 1e-2 + 1e-2 * std::fabs(double(ref[i]))))
            ++r.mismatches;
    }
    r.pass = r.mismatches == 0;
    return r;
}

// ---- results --------------------------------------------------------------------------------
struct Row {
    Case        tc;
    std::string backend, check, detail;
    double      ms = NAN, tflops = NAN, max_abs = NAN;
};

std::string quote(const std::string &s) {
    std::string q = "\"";
    for (const char c : s)
        q += c == '"' ? std::string("\"\"") : std::string(1, c);
    return q + "\"";
}

void write_csv(const std::string &path, const std::vector<Row> &rows, const std::string &gpu, DType dt) {
    std::ofstream f(path);
    if (!f) {
        std::cerr << "error: cannot write " << path << "\n";
        std::exit(1);
    }
    f << "TestID,Case,B,M,N,K,Dtype,GPU,Backend,Check,Time_ms,TFLOPS,MaxAbsErr,Detail\n" << std::fixed;
    for (const auto &r : rows) {
        f << r.tc.id << ',' << r.tc.name << ',' << r.tc.b << ',' << r.tc.m << ',' << r.tc.n << ',' << r.tc.k
          << ',' << dtype_name(dt) << ',' << quote(gpu) << ',' << r.backend << ',' << r.check << ',';
        if (std::isnan(r.ms))
            f << ",,";
        else
            f << std::setprecision(4) << r.ms << ',' << std::setprecision(2) << r.tflops << ',';
        if (!std::isnan(r.max_abs))
            f << std::setprecision(4) << r.max_abs;
        f << ',' << quote(r.detail) << '\n';
    }
}

// Mean time / TFLOPS per backend over the cases every backend passed, and the geometric
// mean of time ratios against the first backend.
void print_summary(const std::vector<Row> &rows, const std::vector<std::string> &backends) {
    std::map<int, std::map<std::string, const Row *>> by_case;
    for (const auto &r : rows)
        by_case[r.tc.id][r.backend] = &r;
    std::vector<int> common;
    for (const auto &[id, m] : by_case) {
        bool all = m.size() == backends.size();
        for (const auto &[b, r] : m)
            all = all && r->check == "PASS";
        if (all)
            common.push_back(id);
    }
    std::cout << "\n==== Summary over " << common.size() << " of " << by_case.size()
              << " cases where all backends passed ====\n";
    if (common.empty())
        return;
    const std::string &ref = backends.front();
    std::cout << std::left << std::setw(20) << "backend" << std::right << std::setw(12) << "sum ms"
              << std::setw(14) << "mean TFLOPS" << std::setw(22) << ("geomean vs " + ref) << std::setw(8)
              << "wins" << '\n';
    for (const auto &b : backends) {
        double sum_ms = 0, sum_tf = 0, lr = 0;
        int    wins   = 0;
        for (const int id : common) {
            const Row *r = by_case[id][b];
            sum_ms += r->ms;
            sum_tf += r->tflops;
            lr += std::log(r->ms / by_case[id][ref]->ms);
            bool best = true;
            for (const auto &o : backends)
                best = best && (o == b || r->ms <= by_case[id][o]->ms);
            wins += best;
        }
        std::cout << std::left << std::setw(20) << b << std::right << std::fixed << std::setprecision(3)
                  << std::setw(12) << sum_ms << std::setprecision(1) << std::setw(14) << sum_tf / common.size()
                  << std::setprecision(3) << std::setw(21) << std::exp(lr / common.size()) << "x" << std::setw(8)
                  << wins << '\n';
    }
    std::cout << "(geomean = time / " << ref << " time, > 1 is slower; wins = fastest on a case)\n";
}

struct DeviceBuffer {
    void  *ptr   = nullptr;
    size_t bytes = 0;
    void  *get(size_t need) {
        if (need > bytes) {
            if (ptr)
                TUNEMAX_HIP_CHECK(hipFree(ptr));
            TUNEMAX_HIP_CHECK(hipMalloc(&ptr, std::max<size_t>(need, 256)));
            bytes = need;
        }
        return ptr;
    }
    ~DeviceBuffer() {
        if (ptr)
            (void)hipFree(ptr);
    }
};

int run(const Options &opt) {
    hipDeviceProp_t prop;
    TUNEMAX_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
    const std::string gpu = std::string(prop.name) + " (" + prop.gcnArchName + ")";

    std::vector<std::unique_ptr<Backend>> backends;
    for (const auto &b : opt.backends)
        backends.push_back(backend_registry().at(b)());

    std::vector<Case> cases;
    for (const auto &c : read_cases(opt.shapes))
        if (opt.only.empty() || opt.only.count(c.id))
            cases.push_back(c);
    std::string out_path = opt.out;
    if (out_path.empty()) {
        char        ts[32];
        std::time_t now = std::time(nullptr);
        std::strftime(ts, sizeof(ts), "%Y%m%d-%H%M%S", std::localtime(&now));
        std::string stem = opt.shapes.substr(opt.shapes.find_last_of('/') + 1);
        out_path = "results_" + stem.substr(0, stem.find_last_of('.')) + "_" + dtype_name(opt.dtype) + "_" + ts + ".csv";
    }
    std::cout << "GPU: " << gpu << "\nshapes: " << opt.shapes << " (" << cases.size() << " cases), dtype "
              << dtype_name(opt.dtype) << ", warmup " << opt.warmup << ", iters " << opt.iters << std::endl;

    hipStream_t stream;
    TUNEMAX_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    hipEvent_t start, stop;
    TUNEMAX_HIP_CHECK(hipEventCreate(&start));
    TUNEMAX_HIP_CHECK(hipEventCreate(&stop));
    DeviceBuffer     xb, wb, ob;
    int64_t         *lens_pinned = nullptr;
    size_t           lens_cap    = 0;
    std::vector<Row> rows;
    const int        gdt = opt.dtype == DType::BF16 ? GG_DTYPE_BF16 : GG_DTYPE_FP16;

    for (const auto &tc : cases) {
        GroupedGemmProblem p;
        p.dtype     = opt.dtype;
        p.group_num = int(tc.b);
        p.n         = tc.n;
        p.k         = tc.k;
        p.group_m.assign(tc.b, tc.m); // balanced groups
        const size_t es = dtype_bytes(p.dtype);
        p.x   = xb.get(size_t(p.total_m()) * p.k * es);
        p.w   = wb.get(size_t(p.group_num) * p.n * p.k * es);
        p.out = ob.get(size_t(p.total_m()) * p.n * es);
        if (lens_cap < size_t(p.group_num)) {
            if (lens_pinned)
                TUNEMAX_HIP_CHECK(hipHostFree(lens_pinned));
            TUNEMAX_HIP_CHECK(hipHostMalloc(&lens_pinned, p.group_num * sizeof(int64_t)));
            lens_cap = p.group_num;
        }
        std::copy(p.group_m.begin(), p.group_m.end(), lens_pinned);
        p.group_lens_pinned = lens_pinned;
        if (gg_fill_randn(gdt, const_cast<void *>(p.x), size_t(p.total_m()) * p.k, 1, stream) != GG_OK ||
            gg_fill_randn(gdt, const_cast<void *>(p.w), size_t(p.group_num) * p.n * p.k, 2, stream) != GG_OK) {
            std::cerr << "fill failed: " << gg_last_error() << "\n";
            return 1;
        }
        const std::vector<Sample> samples = make_samples(p);
        std::cout << "\n[" << tc.id << "] " << tc.name << "  B=" << tc.b << " M=" << tc.m << " N=" << tc.n
                  << " K=" << tc.k << "  (" << std::setprecision(4) << p.flops() / 1e12 << " TFLOP)" << std::endl;

        for (auto &backend : backends) {
            Row row{tc, backend->name(), "", "", NAN, NAN, NAN};
            const auto t_case = std::chrono::steady_clock::now();
            auto       phase  = [&](const char *what) {
                if (opt.verbose)
                    std::cerr << "    [" << tc.id << " " << backend->name() << "] " << what << " at "
                              << std::chrono::duration<double>(std::chrono::steady_clock::now() - t_case).count()
                              << " s" << std::endl;
            };
            try {
                TUNEMAX_HIP_CHECK(hipMemsetAsync(p.out, 0, size_t(p.total_m()) * p.n * es, stream));
                const std::string why = backend->prepare(p, stream);
                if (!why.empty()) {
                    row.check  = "N/A";
                    row.detail = why;
                } else {
                    row.detail = backend->detail();
                    phase("prepared");
                    backend->run(stream);
                    TUNEMAX_HIP_CHECK(hipGetLastError());
                    TUNEMAX_HIP_CHECK(hipStreamSynchronize(stream));
                    phase("first run");
                    if (opt.check) {
                        const CheckResult c = check_output(p, samples, stream);
                        row.check           = c.pass ? "PASS" : "FAIL";
                        row.max_abs         = c.max_abs;
                        if (!c.pass)
                            row.detail += " | " + std::to_string(c.mismatches) + "/" +
                                          std::to_string(samples.size()) + " samples off";
                    } else {
                        row.check = "SKIP";
                    }
                    phase("checked");
                    for (int i = 0; i < opt.warmup; ++i)
                        backend->run(stream);
                    if (opt.verbose)
                        TUNEMAX_HIP_CHECK(hipStreamSynchronize(stream));
                    phase("warmed up");
                    TUNEMAX_HIP_CHECK(hipEventRecord(start, stream));
                    for (int i = 0; i < opt.iters; ++i)
                        backend->run(stream);
                    TUNEMAX_HIP_CHECK(hipEventRecord(stop, stream));
                    TUNEMAX_HIP_CHECK(hipEventSynchronize(stop));
                    TUNEMAX_HIP_CHECK(hipGetLastError());
                    float total = 0.f;
                    TUNEMAX_HIP_CHECK(hipEventElapsedTime(&total, start, stop));
                    row.ms     = double(total) / opt.iters;
                    row.tflops = p.flops() / (row.ms * 1e-3) / 1e12;
                }
            } catch (const std::exception &e) {
                (void)hipStreamSynchronize(stream);
                row.check  = "ERROR";
                row.detail = e.what();
            }
            backend->release();
            std::cout << "  " << std::left << std::setw(18) << row.backend << std::setw(6) << row.check << std::right
                      << std::fixed;
            if (std::isnan(row.ms))
                std::cout << std::setw(12) << "-" << std::setw(14) << "-";
            else
                std::cout << std::setprecision(4) << std::setw(10) << row.ms << " ms" << std::setprecision(1)
                          << std::setw(9) << row.tflops << " TFLOPS";
            std::cout << "  " << row.detail.substr(0, 90) << std::endl;
            std::cout.unsetf(std::ios::fixed);
            rows.push_back(row);
        }
        write_csv(out_path, rows, gpu, opt.dtype); // after every case: a crash keeps the rest
    }
    print_summary(rows, opt.backends);
    std::cout << "\nresults: " << out_path << "\n";
    if (lens_pinned)
        TUNEMAX_HIP_CHECK(hipHostFree(lens_pinned));
    TUNEMAX_HIP_CHECK(hipEventDestroy(start));
    TUNEMAX_HIP_CHECK(hipEventDestroy(stop));
    TUNEMAX_HIP_CHECK(hipStreamDestroy(stream));
    for (const auto &r : rows)
        if (r.check == "FAIL" || r.check == "ERROR")
            return 1;
    return 0;
}

} // namespace
} // namespace tunemax

int main(int argc, char **argv) { return tunemax::run(tunemax::parse_args(argc, argv)); }
