// extern "C" boundary of the grouped GEMM (declared in include/gg_grouped_gemm.h).
//
// Host side of the reference's ck_tile backend, redone for the hand-written gfx950 kernel:
// CkTileBackend::prepare_typed / finish / run / release (ck_kernel/ck_grouped_gemm.cpp:126-226).
// prepare validates the problem, builds the device group table (row offset, rows, first
// tile per group) and the launch shape; run enqueues one launch and never synchronizes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "gg_grouped_gemm.h"
#include "gg_kernel.h"

struct gg_plan {
    int                 mode        = 0; // 0 forward, 1 dgrad, 2 wgrad (kernel terms: KernelArgs)
    int                 dtype       = GG_DTYPE_BF16;
    int                 group_num   = 0;
    int64_t             n           = 0;
    int64_t             k           = 0;
    int64_t             total_m     = 0;
    int                 total_tiles = 0;
    int                 grid        = 0;
    const void         *x           = nullptr;
    const void         *w           = nullptr;
    void               *out         = nullptr;
    gg::GroupEntry     *d_groups    = nullptr;
    gg::KernelArgs      args{};
    std::string         detail;
    // Device-resident group sizes (gg_prepare_device_lens): the table is rebuilt per run.
    bool                device_lens = false;
    const int64_t      *d_lens      = nullptr;
    const int64_t      *d_offs      = nullptr;
    gg::TableHeader    *d_header    = nullptr; // follows the table in the d_groups allocation
    bool                in_kernel_table = false; // the GEMM builds the table (no table launch)
    float              *d_ws        = nullptr; // split-K / tail-split partial sums (args.ws)
    gg::TileDesc       *d_desc      = nullptr; // tile descriptors (args.desc)
    int64_t             in_rows     = 0;       // device-size plans: rows of the inputs
    // Small-tile plans (use_small_tiles): the launch of gg_small.hip instead of the persistent one.
    bool                small       = false;
    gg::SmallArgs       sargs{};
    gg::SmallTile      *d_small     = nullptr; // [sargs.tiles]
};

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string &msg) {
    g_last_error = msg;
    return status;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(GG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// XCDs of the device: MI355X (gfx950) has 8, each with its own L2. Workgroups are
// dispatched round-robin over them.
int xcd_count(const hipDeviceProp_t &prop) {
    const std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) == 0 || arch.rfind("gfx942", 0) == 0)
        return 8;
    return 1;
}

// Shape and pointer rules shared by both prepare entry points; returns GG_OK or a failure.
int check_problem(int dtype, int group_num, int64_t n, int64_t k, bool has_output, const void *x,
                  const void *w, const void *out) {
    if (dtype != GG_DTYPE_BF16 && dtype != GG_DTYPE_FP16)
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_BF16 or GG_DTYPE_FP16");
    if (group_num < 0 || n < 0 || k < 0)
        return fail(GG_ERR_INVALID, "group_num, n and k must be >= 0");
    if (has_output && (out == nullptr || (k > 0 && (x == nullptr || w == nullptr))))
        return fail(GG_ERR_INVALID, "x, w and out must be device pointers");
    // Shapes the kernel cannot take: reported like a non-empty Backend::prepare result.
    if (n % 8 != 0)
        return fail(GG_ERR_UNSUPPORTED, "N must be a multiple of 8 (16-byte output rows)");
    if (k % 8 != 0)
        return fail(GG_ERR_UNSUPPORTED, "K must be a multiple of 8 (16-byte input rows)");
    if (has_output && (!aligned16(out) || (k > 0 && (!aligned16(x) || !aligned16(w)))))
        return fail(GG_ERR_UNSUPPORTED, "x, w and out must be 16-byte aligned");
    // 32-bit per-tile byte offsets: a 256-row slice of x, w or out must stay below 2 GiB.
    if (k > (int64_t(1) << 21) || n > (int64_t(1) << 21))
        return fail(GG_ERR_UNSUPPORTED, "N and K must be at most 2097152");
    return GG_OK;
}

int device_props(hipDeviceProp_t *prop) {
    int        dev = 0;
    hipError_t e   = hipGetDevice(&dev);
    if (e == hipSuccess)
        e = hipGetDeviceProperties(prop, dev);
    return e == hipSuccess ? GG_OK : hip_fail(e, "hipGetDeviceProperties");
}

void fill_args(gg_plan *plan, int n_xcd) {
    gg::KernelArgs &a = plan->args;
    a.x         = plan->x;
    a.w         = plan->w;
    a.out       = plan->out;
    a.groups    = plan->d_groups;
    a.group_num = plan->group_num;
    a.n         = static_cast<int>(plan->n);
    a.k         = static_cast<int>(plan->k);
    a.n_tiles   = static_cast<int>(gg::cdiv(plan->n, gg::kTileN));
    a.k_tiles   = static_cast<int>(gg::cdiv(plan->k, gg::kTileK));
    a.n_xcd     = plan->grid % n_xcd == 0 ? n_xcd : 1;
    a.band      = gg::band_for(plan->n, plan->k, plan->mode / 4 == gg::kIn16 ? 2 : 1);
    // GG_BAND=<1..64> in the environment overrides the M-tiles per band of the in-group order
    // (measurements only)
    if (const char *env = std::getenv("GG_BAND"); env != nullptr && std::atoi(env) >= 1 && std::atoi(env) <= 64)
        a.band = std::atoi(env);
    a.lda       = static_cast<int>(plan->k);
    a.ldb       = static_cast<int>(plan->k);
    a.m_out     = 0;
    a.min_steps = 0;
    a.x_scale   = nullptr;
    a.w_scale   = nullptr;
    a.splits    = 1;
    a.ws        = nullptr;
    a.tile_n    = gg::kTileN;
    a.tile_m    = gg::kTileM;
    a.tail_splits = 1;
    a.desc        = nullptr;
    a.desc_per_wg = 0;
    a.tails       = 1; // set by the plan builders that know the sizes
}

// Split-K for problems whose tiles cannot fill the GPU (fewer than half as many tiles as CUs):
// each tile's K steps are cut into S ranges computed by different workgroups, which write fp32
// partial sums (256 KB per unit) that a second kernel adds in split order (deterministic) and
// converts. S minimises a launch-time model, in microseconds, fitted to MI355X timings of
// one-round problems (24-64 tiles, 22-256 K steps):
//   S = 1: k_tiles * kStepUs (one round of tiles)
//   S > 1: ceil(k_tiles / S) * kStepUs + kSplitUs + S * tiles * kSlabUs
// within one round (S * tiles <= CUs) and at least kMinSplitSteps K steps per range, taken only
// when it predicts at least kMinSplitGain (the cost of the partial sums grows faster than
// linearly near a full round of units, so small predicted gains are often losses).
// GG_SPLIT_K=<S> in the environment forces S (clamped to [1, k_tiles]; 1 turns split-K off).
constexpr double kStepUs        = 1.2;  // one K step of a 256 x 256 tile
constexpr double kSplitUs       = 3.0;  // second launch and its latency
constexpr double kSlabUs        = 0.15; // one unit's 256 KB of partial sums, written and read back
constexpr int    kMinSplitSteps = 4;
constexpr double kMinSplitGain  = 0.15;

int choose_splits(int tiles, int k_tiles, int cus) {
    if (const char *env = std::getenv("GG_SPLIT_K")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1)
            return static_cast<int>(std::min<long>(v, k_tiles));
    }
    const int max_s = std::min(cus / std::max(tiles, 1), k_tiles / kMinSplitSteps);
    const double unsplit = k_tiles * kStepUs;
    int          best    = 1;
    double       cost    = unsplit;
    for (int sp = 2; sp <= max_s; ++sp) {
        const double c = ((k_tiles + sp - 1) / sp) * kStepUs + kSplitUs + double(sp) * tiles * kSlabUs;
        if (c < cost) {
            cost = c;
            best = sp;
        }
    }
    return cost <= (1.0 - kMinSplitGain) * unsplit ? best : 1;
}

// Narrow tiles (256 x 224) for a forward plan of one round that leaves CUs idle: when the plan is
// not split and the 224-wide tiling still fits in one round, it gives more workgroups 7/8 of a
// tile each (1 x 2048 x 7168: 224 tiles of 256 x 256 on 256 CUs, 256 tiles of 256 x 224). The
// group table is rebuilt for the narrow tile count. GG_NARROW=0 in the environment turns this
// off.
int use_narrow_tiles(gg_plan *plan, const int64_t *group_m, const hipDeviceProp_t &prop, hipStream_t s) {
    gg::KernelArgs &a   = plan->args;
    const char     *env = std::getenv("GG_NARROW");
    if ((env != nullptr && *env != '\0' && std::atoi(env) == 0) || a.splits > 1 || a.tile_m != gg::kTileM ||
        plan->total_tiles >= prop.multiProcessorCount)
        return GG_OK;
    const int64_t               n_tiles = gg::cdiv(plan->n, gg::kNarrowTileN);
    std::vector<gg::GroupEntry> table(static_cast<size_t>(plan->group_num));
    const int64_t tiles = gg::build_group_table(group_m, plan->group_num, n_tiles, table.data());
    if (tiles <= plan->total_tiles || tiles > prop.multiProcessorCount)
        return GG_OK;
    hipError_t e = hipMemcpyAsync(plan->d_groups, table.data(), table.size() * sizeof(gg::GroupEntry),
                                  hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e != hipSuccess)
        return hip_fail(e, "narrow group table upload");
    plan->total_tiles = static_cast<int>(tiles);
    plan->grid        = plan->total_tiles;
    a.total_tiles     = plan->total_tiles;
    a.n_tiles         = static_cast<int>(n_tiles);
    a.tile_n          = gg::kNarrowTileN;
    const int n_xcd   = xcd_count(prop);
    a.n_xcd           = plan->grid % n_xcd == 0 ? n_xcd : 1;
    return GG_OK;
}

// Modelled time, in full 256 x 256 tile steps, of the busiest workgroup when tiles of tile_m rows
// are dealt to the grid in the kernel's order (xcd_remap over the group table's banded order).
// A tile's cost by its valid rows m, fitted to MI355X timings of partial tiles (one launch
// per row count, 256 groups, cross-tile): with 256-row tiles 1 for a full tile, 0.86-1 for
// 129-255 rows, and 0.70-0.85 for at most 128 rows (thin steps); with short tiles (at most 192
// rows, six row blocks per wave) the same below 129 rows and 0.85-0.88 above.
double busiest_workgroup(const int64_t *group_m, int group_num, int64_t n_tiles, int tile_m, int tiles,
                         int grid, int n_xcd, int band) {
    std::vector<float> cost(static_cast<size_t>(tiles));
    int                L = 0;
    for (int g = 0; g < group_num; ++g) {
        const int m_tiles = static_cast<int>(gg::cdiv(group_m[g], tile_m));
        for (int local = 0; local < m_tiles * n_tiles; ++local, ++L) {
            int tm, tn;
            gg::band_coords(local, m_tiles, static_cast<int>(n_tiles), band, &tm, &tn);
            const double m = static_cast<double>(std::min<int64_t>(tile_m, group_m[g] - int64_t(tm) * tile_m));
            double       c;
            if (m <= 128)
                c = 0.70 + 0.15 * m / 128;
            else if (tile_m < gg::kTileM)
                c = 0.85 + 0.03 * (m - 128) / 64;
            else
                c = m >= gg::kTileM ? 1.0 : 0.86 + 0.14 * (m - 128) / 128;
            cost[static_cast<size_t>(L)] = static_cast<float>(c);
        }
    }
    std::vector<double> load(static_cast<size_t>(grid), 0.0);
    for (int t = 0; t < tiles; ++t)
        load[static_cast<size_t>(t % grid)] += cost[static_cast<size_t>(gg::xcd_remap(t, tiles, grid, n_xcd))];
    return *std::max_element(load.begin(), load.end());
}

// Short tiles (at most 192 x 256) for a 16-bit forward or dgrad plan whose groups keep their M-tile
// counts with fewer rows per tile (gg::short_tile_rows): the same tiles, and the same total
// loads, but no group ends in a nearly empty tile next to full ones. Taken when the modelled
// busiest workgroup is at least 3 % faster (32 groups of 520 rows, N = K = 2880: three tiles of
// 176 rows per group; 4.71 -> 4.36 tile steps). The group table is rebuilt for the tile rows.
// GG_SHORT=0 in the environment turns this off, GG_SHORT=1 takes short tiles whenever the tile
// counts allow.
int use_short_tiles(gg_plan *plan, const int64_t *group_m, hipStream_t s) {
    gg::KernelArgs &a   = plan->args;
    const char     *env = std::getenv("GG_SHORT");
    const int       opt = env != nullptr && *env != '\0' ? std::atoi(env) : -1;
    if (opt == 0 || a.splits > 1 || a.tile_n != gg::kTileN)
        return GG_OK;
    const int rows = gg::short_tile_rows(group_m, plan->group_num);
    if (rows <= 0)
        return GG_OK;
    if (opt != 1) {
        const double wide  = busiest_workgroup(group_m, plan->group_num, a.n_tiles, gg::kTileM,
                                               plan->total_tiles, plan->grid, a.n_xcd, a.band);
        const double short_ = busiest_workgroup(group_m, plan->group_num, a.n_tiles, rows,
                                                plan->total_tiles, plan->grid, a.n_xcd, a.band);
        if (short_ > 0.97 * wide)
            return GG_OK;
    }
    std::vector<gg::GroupEntry> table(static_cast<size_t>(plan->group_num));
    const int64_t tiles = gg::build_group_table(group_m, plan->group_num, a.n_tiles, table.data(), 0, rows);
    if (tiles != plan->total_tiles)
        return fail(GG_ERR_INVALID, "short tiles changed the tile count");
    hipError_t e = hipMemcpyAsync(plan->d_groups, table.data(), table.size() * sizeof(gg::GroupEntry),
                                  hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e != hipSuccess)
        return hip_fail(e, "short group table upload");
    a.tile_m = rows;
    return GG_OK;
}

// Short-wide tiles (at most 192 x 288) for a cross-tile 16-bit forward plan of short tiles: nine
// column blocks per wave instead of eight, so the same loads per K step feed 9/8 of the MFMAs and
// fewer tiles make fewer rounds (32 groups of 520 rows, N = K = 2880: 1152 short tiles, 4.5
// rounds on 256 CUs; 960 short-wide tiles, 3.75 rounds, and no 64-column tail tile). A
// short-wide tile is modelled at kWideTileCost short tiles (its K step moves 7 % more bytes for
// 12.5 % more MFMAs); taken when the modelled busiest workgroup gains at least 5 % and the plan
// stays cross-tile. The group table is rebuilt for the 288-column tiles.
// GG_WIDE=0 in the environment turns this off, GG_WIDE=1 takes short-wide tiles wherever the
// plan allows them.
constexpr double kWideTileCost = 1.10;

int use_short_wide_tiles(gg_plan *plan, const int64_t *group_m, const hipDeviceProp_t &prop, hipStream_t s) {
    gg::KernelArgs &a   = plan->args;
    const char     *env = std::getenv("GG_WIDE");
    const int       opt = env != nullptr && *env != '\0' ? std::atoi(env) : -1;
    if (opt == 0 || plan->mode != gg::make_mode(gg::kFwd, gg::kIn16) || a.tile_m == gg::kTileM ||
        a.tile_n != gg::kTileN || a.splits > 1 || a.d_total != nullptr || a.d_lens != nullptr)
        return GG_OK;
    const int64_t n_tiles = gg::cdiv(plan->n, gg::kShortWideTileN);
    std::vector<gg::GroupEntry> table(static_cast<size_t>(plan->group_num));
    const int64_t tiles = gg::build_group_table(group_m, plan->group_num, n_tiles, table.data(), 0, a.tile_m);
    if (tiles <= 0 || tiles > INT32_MAX)
        return GG_OK;
    const int grid  = static_cast<int>(std::min<int64_t>(prop.multiProcessorCount, tiles));
    const int n_xcd = grid % xcd_count(prop) == 0 ? xcd_count(prop) : 1;
    gg::KernelArgs w = a;
    w.total_tiles    = static_cast<int>(tiles);
    w.n_tiles        = static_cast<int>(n_tiles);
    w.tile_n         = gg::kShortWideTileN;
    w.n_xcd          = n_xcd;
    if (!gg::uses_cross_tile(w, grid, plan->mode))
        return GG_OK;
    if (opt != 1) {
        const double short_ = busiest_workgroup(group_m, plan->group_num, a.n_tiles, a.tile_m, plan->total_tiles,
                                                plan->grid, a.n_xcd, a.band);
        const double wide   = kWideTileCost * busiest_workgroup(group_m, plan->group_num, n_tiles, a.tile_m,
                                                                w.total_tiles, grid, n_xcd, a.band);
        if (wide > 0.95 * short_)
            return GG_OK;
    }
    hipError_t e = hipMemcpyAsync(plan->d_groups, table.data(), table.size() * sizeof(gg::GroupEntry),
                                  hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e != hipSuccess)
        return hip_fail(e, "short-wide group table upload");
    plan->total_tiles = w.total_tiles;
    plan->grid        = grid;
    a                 = w;
    return GG_OK;
}

// Picks the plan's split count (plan->args filled, k_tiles set) and allocates the partial sums.
int setup_split_k(gg_plan *plan, const hipDeviceProp_t &prop) {
    gg::KernelArgs &a  = plan->args;
    const int       sp = choose_splits(plan->total_tiles, a.k_tiles, prop.multiProcessorCount);
    if (sp <= 1)
        return GG_OK;
    const size_t bytes = size_t(sp) * size_t(plan->total_tiles) * 262144;
    const hipError_t e = hipMalloc(&plan->d_ws, bytes);
    if (e != hipSuccess)
        return hip_fail(e, "split-K workspace allocation");
    a.splits    = sp;
    a.ws        = plan->d_ws;
    plan->grid  = static_cast<int>(std::min<int64_t>(prop.multiProcessorCount, int64_t(sp) * plan->total_tiles));
    return GG_OK;
}

// Tail split for cross-tile 16-bit forward plans (host-size tables): when the last round holds
// rem tiles, at most half the grid, each of them is cut into two K ranges run by two workgroups,
// so the busiest workgroup does R + 1/2 tiles instead of R + 1 (R full rounds). The ranges store
// fp32 partial sums (2 * rem slabs of 256 KB) and tail_reduce_kernel, launched right after the
// GEMM on the same stream, adds and stores them. Taken when a launch-time model (microseconds,
// fitted to MI355X end-to-end timings) predicts a gain: the busiest workgroup saves T / 2 K steps
// (kStepUs each), and pays its 256 KB of partial sums through the store path (kTailStoreUs), the
// second launch (kTailLaunchUs) and the reduction's traffic, 1.5 MB per last-round tile
// (kTailTileUs). Measured: 3 x 4096 x 1536 x 2048 (32 tiles in the last round, 32 K steps) 935 ->
// 980 TFLOPS; config 5a (128 tiles, 45 steps) 1022 -> 948 and 1 x 4096 x 5376 x 2048 (80 tiles)
// 1097 -> 1030, both left unsplit by the model. At least kMinTailSteps K steps per range.
// GG_TAIL_SPLIT=0 in the environment turns it off; GG_TAIL_SPLIT=2 takes it wherever the plan
// allows a split.
constexpr int    kMinTailSteps = 8;
constexpr double kTailStoreUs  = 6.0;
constexpr double kTailLaunchUs = 5.0;
constexpr double kTailTileUs   = 0.15;

int setup_tail_split(gg_plan *plan) {
    gg::KernelArgs &a = plan->args;
    a.tail_splits     = 1;
    if (plan->mode != gg::make_mode(gg::kFwd, gg::kIn16) || a.splits > 1 || a.d_total != nullptr ||
        a.d_lens != nullptr || a.tile_n != gg::kTileN || !gg::uses_cross_tile(a, plan->grid, plan->mode))
        return GG_OK;
    const int grid = plan->grid, tiles = plan->total_tiles;
    const int full = tiles / grid * grid, rem = tiles - full;
    if (full == 0 || rem == 0 || 2 * rem > grid)
        return GG_OK;
    int forced = -1;
    if (const char *env = std::getenv("GG_TAIL_SPLIT"); env != nullptr && *env != '\0')
        forced = std::atoi(env);
    if (forced == 0 || forced == 1)
        return GG_OK;
    constexpr int sp = 2;
    if (a.k_tiles / sp < (forced > 1 ? gg::kCrossMinStepsHost : kMinTailSteps))
        return GG_OK;
    const double saved_us = (a.k_tiles - gg::cdiv(a.k_tiles, sp)) * kStepUs;
    const double cost_us  = kTailStoreUs + kTailLaunchUs + rem * kTailTileUs;
    if (forced < 0 && saved_us < 1.1 * cost_us)
        return GG_OK;
    const hipError_t e = hipMalloc(&plan->d_ws, size_t(rem) * size_t(sp) * 262144);
    if (e != hipSuccess)
        return hip_fail(e, "tail-split workspace");
    a.tail_splits = sp;
    a.ws          = plan->d_ws;
    return GG_OK;
}

// Small tiles (128 x 128, one per workgroup, gg_small.hip) for 16-bit forward plans of host-size
// groups whose 256 x 256 tiles fill at most half the CUs (one round of the per-tile variant).
// The small-tile kernel runs its K steps at about half the MFMA rate of the persistent kernel
// (twice the LDS reads per MFMA) but brings about four times the workgroups. Taken when its
// tiles (unsplit unless GG_SMALL_SPLIT says otherwise) fit two per CU and a launch-time model
// (microseconds, MI355X) predicts at most kSmallGain of the persistent plan's time:
// kSmallFixedUs + K steps * kSmallStepUs (one workgroup per CU, a 4-step ring) or
// kSmallStepTwoUs (up to two, a 2-step ring) against kSmallFixedUs + the split-K model of
// choose_splits for the plan's own splits. Against GG_SMALL=0 (gg_bench and ab runs, bf16): one
// per CU, the suite's TestIDs 109, 110, 112, 122, 157, 160, 170 and 194 1.23-1.49x, pad_test's
// 9002 and 9004 and config 1; two per CU, 1 x 2048 x 2880 x 2880 1.13x, 1 x 1024 x 5760 x 2880
// 1.05x, 2 x 1024 x 2816 x 2048 1.03x. Left out: where the persistent plan splits a long K
// (146, 266, 268, 278, 148: small tiles 0.63-0.78x) and more than two tiles per CU.
// For forced plans (GG_SMALL=1) the K ranges fill up to one workgroup per CU (128 KB of LDS
// each) with at least kMinSmallSteps K steps per range; they write fp32 partial sums (64 KB per
// tile and range) that a second launch adds in range order. GG_SMALL=0 in the environment turns
// small tiles off; GG_SMALL_SPLIT=<S> forces the ranges.
constexpr int    kMinSmallSteps = 8;
constexpr double kSmallFixedUs  = 4.0;  // launch, first DMAs, epilogue
constexpr double kSmallStepUs    = 0.62; // one K step of a 128 x 128 tile, one workgroup per CU
constexpr double kSmallStepTwoUs = 1.0;  // the same with up to two workgroups per CU
constexpr double kSmallGain      = 0.85;

int use_small_tiles(gg_plan *plan, const int64_t *group_m, const hipDeviceProp_t &prop, hipStream_t s) {
    const char *env = std::getenv("GG_SMALL");
    const int   opt = env != nullptr && *env != '\0' ? std::atoi(env) : -1;
    const int   cus = prop.multiProcessorCount;
    const gg::KernelArgs &a = plan->args;
    if (opt == 0 || plan->group_num > 32767 || (opt != 1 && (2 * plan->total_tiles > cus || a.tail_splits > 1)))
        return GG_OK;
    const int64_t              nt = gg::cdiv(plan->n, gg::kSmallTile);
    std::vector<gg::SmallTile> list;
    int64_t                    row = 0;
    for (int g = 0; g < plan->group_num; ++g) {
        const int64_t mt = gg::cdiv(group_m[g], gg::kSmallTile);
        for (int64_t tn = 0; tn < nt; ++tn)
            for (int64_t tm = 0; tm < mt; ++tm)
                list.push_back({row + tm * gg::kSmallTile,
                                static_cast<int32_t>(std::min<int64_t>(gg::kSmallTile, group_m[g] - tm * gg::kSmallTile)),
                                static_cast<int16_t>(g), static_cast<int16_t>(tn)});
        row += group_m[g];
    }
    const int64_t tiles   = static_cast<int64_t>(list.size());
    const int     k_steps = static_cast<int>(gg::cdiv(plan->k, gg::kSmallK));
    if (tiles == 0 || tiles > 65536)
        return GG_OK;
    // Workgroup i runs on XCD i % n_xcd: deal the list (N-tile by N-tile, M-tiles inside) to the
    // XCDs in contiguous runs (xcd_remap), so that the workgroups of one XCD share a few x and w
    // panels in its L2 instead of every XCD reading every w panel.
    // (A grid of whole XCD rows: XCD y takes ceil((tiles - y) / n_xcd) of the list.)
    if (const int n_xcd = xcd_count(prop); n_xcd > 1) {
        const int                  rows = static_cast<int>(gg::cdiv(tiles, n_xcd)) * n_xcd;
        std::vector<gg::SmallTile> dealt(list.size());
        for (int t = 0; t < static_cast<int>(tiles); ++t)
            dealt[static_cast<size_t>(t)] = list[static_cast<size_t>(gg::xcd_remap(t, static_cast<int>(tiles), rows, n_xcd))];
        list.swap(dealt);
    }
    int sp = 1;
    if (opt == 1 && tiles < cus) // forced: fill the CUs with K ranges
        sp = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(cus / tiles, k_steps / kMinSmallSteps)));
    if (const char *e2 = std::getenv("GG_SMALL_SPLIT"); e2 != nullptr && std::atoi(e2) >= 1)
        sp = std::min(std::atoi(e2), k_steps);
    const int per = static_cast<int>(gg::cdiv(k_steps, sp));
    sp            = static_cast<int>(gg::cdiv(k_steps, per)); // no empty K range
    // a 4-step ring while every workgroup has a CU of its own, else a 2-step ring, two per CU
    const int stages = tiles * sp <= cus ? gg::kSmallStagesOne : gg::kSmallStagesTwo;
    if (opt != 1) {
        const double big   = kSmallFixedUs + gg::cdiv(a.k_tiles, a.splits) * kStepUs +
                           (a.splits > 1 ? kSplitUs + double(a.splits) * plan->total_tiles * kSlabUs : 0.0);
        const double step  = stages == gg::kSmallStagesOne ? kSmallStepUs : kSmallStepTwoUs;
        const double small = kSmallFixedUs + double(per) * step;
        if (tiles * sp > 2 * int64_t(cus) || small > kSmallGain * big)
            return GG_OK;
    }
    // the persistent plan's workspace and descriptors are not used by this launch
    if (plan->d_ws != nullptr)
        (void)hipFree(plan->d_ws);
    if (plan->d_desc != nullptr)
        (void)hipFree(plan->d_desc);
    plan->d_ws   = nullptr;
    plan->d_desc = nullptr;
    const size_t bytes = list.size() * sizeof(gg::SmallTile);
    hipError_t   e     = hipMalloc(&plan->d_small, bytes);
    if (e == hipSuccess)
        e = hipMemcpyAsync(plan->d_small, list.data(), bytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e == hipSuccess && sp > 1)
        e = hipMalloc(&plan->d_ws, size_t(sp) * size_t(tiles) * gg::kSmallTile * gg::kSmallTile * sizeof(float));
    if (e != hipSuccess)
        return hip_fail(e, "small-tile plan");
    gg::SmallArgs &sa    = plan->sargs;
    sa.x                 = plan->x;
    sa.w                 = plan->w;
    sa.out               = plan->out;
    sa.tile_list         = plan->d_small;
    sa.ws                = plan->d_ws;
    sa.tiles             = static_cast<int>(tiles);
    sa.n                 = static_cast<int>(plan->n);
    sa.k                 = static_cast<int>(plan->k);
    sa.k_steps           = k_steps;
    sa.splits            = sp;
    sa.steps_per_split   = per;
    sa.stages            = stages;
    plan->small          = true;
    plan->total_tiles    = static_cast<int>(tiles);
    plan->grid           = static_cast<int>(tiles) * sp;
    return GG_OK;
}

void free_plan(gg_plan *plan) {
    if (plan->d_small != nullptr)
        (void)hipFree(plan->d_small);
    if (plan->d_groups != nullptr)
        (void)hipFree(plan->d_groups);
    if (plan->d_ws != nullptr)
        (void)hipFree(plan->d_ws);
    if (plan->d_desc != nullptr)
        (void)hipFree(plan->d_desc);
    delete plan;
}

// Tile descriptors of forward, dgrad and wgrad plans of whole tiles (host-size tables): every
// workgroup's tiles in the kernel's own walk (xcd_remap, then locate_tile over the plan's group
// table with its tile rows and N-tiles), so that the kernel reads a tile's first row, group and
// N-tile from a lane of a register instead of recomputing them between its K loops. Not built
// (the kernel walks the table itself) with split-K, a tail split, more than kMaxDescPerWg tiles
// per workgroup or rows past 2^31 (output rows, and for wgrad the input tokens whose offsets its
// descriptors hold). GG_TILE_DESC=0 in the environment turns them off.
int setup_tile_desc(gg_plan *plan, const int64_t *group_m, hipStream_t s) {
    gg::KernelArgs &a   = plan->args;
    const char     *env = std::getenv("GG_TILE_DESC");
    if ((env != nullptr && env[0] == '0') || a.splits > 1 || a.tail_splits > 1 || plan->grid <= 0 ||
        !gg::desc_rows_fit(group_m, plan->group_num, plan->total_m))
        return GG_OK;
    const int per_wg = static_cast<int>(gg::cdiv(plan->total_tiles, plan->grid));
    if (per_wg > gg::kMaxDescPerWg)
        return GG_OK;
    // wgrad: every group owns m_out / 256 x N-tiles output tiles whatever its size
    const bool    wgrad    = plan->mode % 4 == gg::kWgrad;
    const int64_t out_rows = wgrad ? a.m_out : 0;
    if (wgrad && (gg::cdiv(out_rows, a.tile_m) > 0xffff || a.n_tiles > 0x7fff))
        return GG_OK;
    std::vector<gg::GroupEntry> table(static_cast<size_t>(plan->group_num));
    const int64_t tiles = gg::build_group_table(group_m, plan->group_num, a.n_tiles, table.data(), out_rows, a.tile_m);
    if (tiles != plan->total_tiles)
        return fail(GG_ERR_INVALID, "tile descriptors: the group table's tile count differs from the plan's");
    std::vector<gg::TileDesc> desc(static_cast<size_t>(plan->grid) * per_wg, gg::TileDesc{0, 0, 0, 0});
    for (int wg = 0; wg < plan->grid; ++wg) {
        int g = 0; // locate_tile's hint: a workgroup's logical tiles only grow
        for (int i = 0; i < per_wg; ++i) {
            const int t = wg + i * plan->grid;
            if (t >= plan->total_tiles)
                break;
            const int L = gg::xcd_remap(t, plan->total_tiles, plan->grid, a.n_xcd);
            int       tm, tn;
            gg::locate_tile(L, table.data(), plan->group_num, a.n_tiles, a.band, &g, &tm, &tn,
                            static_cast<int>(out_rows), a.tile_m);
            if (wgrad) { // the group's first token, (N-tile << 16) | M-tile, the group's tokens
                desc[static_cast<size_t>(wg) * per_wg + i] =
                    gg::TileDesc{static_cast<int32_t>(table[g].row0), g, (tn << 16) | tm, table[g].m};
                continue;
            }
            const int64_t r0 = table[g].row0 + static_cast<int64_t>(tm) * a.tile_m;
            const int     mv = static_cast<int>(std::min<int64_t>(a.tile_m, table[g].m - static_cast<int64_t>(tm) * a.tile_m));
            desc[static_cast<size_t>(wg) * per_wg + i] = gg::TileDesc{static_cast<int32_t>(r0), g, (tn << 9) | mv, 0};
        }
    }
    const size_t bytes = desc.size() * sizeof(gg::TileDesc);
    hipError_t   e     = hipMalloc(&plan->d_desc, bytes);
    if (e == hipSuccess)
        e = hipMemcpyAsync(plan->d_desc, desc.data(), bytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e != hipSuccess)
        return hip_fail(e, "tile descriptor upload");
    a.desc        = reinterpret_cast<const int *>(plan->d_desc);
    a.desc_per_wg = per_wg;
    return GG_OK;
}

} // namespace

namespace {

// ---------------------------------------------------------------------------------------
// Device-resident group sizes: the plan builder shared by gg_prepare_device_lens_op (a plan that
// owns its table, hipMalloc'd) and gg_run_device_lens_noalloc (one call that allocates nothing:
// the table and its header live in the device's `scratch` array below).
// ---------------------------------------------------------------------------------------

// Scratch of the allocation-free entry point: the group table (16 bytes per group) and its
// header. One copy per GPU, held until the process ends; every call on a GPU shares it, so
// calls that overlap on one GPU (two streams, two host threads) race on it. Host code never
// names `scratch` in a kernel argument or copy: it uses the device address that
// hipGetSymbolAddress gives for the current device (noalloc_device).
constexpr int    kNoAllocMaxGroups  = 8192;
constexpr size_t kNoAllocTableBytes = size_t(kNoAllocMaxGroups) * sizeof(gg::GroupEntry);
constexpr size_t kScratchBytes      = kNoAllocTableBytes + 256; // + the TableHeader, padded
static_assert(sizeof(gg::TableHeader) <= 256, "the header fits behind the largest table");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// What the allocation-free entry point keeps per device: the scratch address and the launch
// facts of hipGetDeviceProperties (queried once, not per call).
struct NoAllocDevice {
    void *scratch = nullptr;
    int   cus     = 0;
    int   n_xcd   = 1;
};
constexpr int kNoAllocMaxDevices = 64;
std::mutex    g_noalloc_mu;
NoAllocDevice g_noalloc_dev[kNoAllocMaxDevices];

// The current device's entry, set up on its first use with that device current.
int noalloc_device(NoAllocDevice *out) {
    int        dev = 0;
    hipError_t e   = hipGetDevice(&dev);
    if (e != hipSuccess)
        return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kNoAllocMaxDevices)
        return fail(GG_ERR_UNSUPPORTED, "device index " + std::to_string(dev) + " beyond " +
                                            std::to_string(kNoAllocMaxDevices));
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    NoAllocDevice              &d = g_noalloc_dev[dev];
    if (d.scratch == nullptr) {
        hipDeviceProp_t prop;
        if (device_props(&prop) != GG_OK)
            return GG_ERR_HIP;
        void *p = nullptr;
        e       = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
            return fail(GG_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null or misaligned address");
        d.cus     = prop.multiProcessorCount;
        d.n_xcd   = xcd_count(prop);
        d.scratch = p;
    }
    *out = d;
    return GG_OK;
}

// Validates a device-size problem (the rules of gg_prepare_device_lens_op) and fills *plan.
// noalloc = false: the table and header are one hipMalloc owned by the plan (free_plan releases
// it, also on failure). noalloc = true: they are the current device's scratch array, and nothing
// is allocated (no detail text either). A plan without a launch keeps d_groups null.
int plan_device_lens(gg_plan *plan, bool noalloc, int op, int a_dtype, int b_dtype, int group_num,
                     int64_t total_m, int64_t n, int64_t k, const int64_t *group_lens, const int64_t *group_offs,
                     const void *a, const void *b, const float *a_scale, const float *b_scale, void *out) {
    if (op != GG_OP_FORWARD && op != GG_OP_DGRAD && op != GG_OP_WGRAD)
        return fail(GG_ERR_INVALID, "op must be GG_OP_FORWARD, GG_OP_DGRAD or GG_OP_WGRAD");
    if (total_m < 0 || group_num < 0 || n < 0 || k < 0)
        return fail(GG_ERR_INVALID, "group_num, total_m, n and k must be >= 0");
    if (group_num > 0 && group_lens == nullptr)
        return fail(GG_ERR_INVALID, "group_lens is null");
    // Input formats: two equal 16-bit types, or fp8 (forward: both e4m3 or both e5m2; backward
    // also an e5m2 gradient with e4m3 w / x).
    const bool f8     = a_dtype == GG_DTYPE_FP8_E4M3 || a_dtype == GG_DTYPE_FP8_E5M2;
    int        format = gg::kIn16;
    if (f8) {
        if (a_dtype == GG_DTYPE_FP8_E4M3 && b_dtype == GG_DTYPE_FP8_E4M3)
            format = gg::kInE4M3;
        else if (a_dtype == GG_DTYPE_FP8_E5M2 && b_dtype == GG_DTYPE_FP8_E5M2)
            format = gg::kInE5M2;
        else if (op != GG_OP_FORWARD && a_dtype == GG_DTYPE_FP8_E5M2 && b_dtype == GG_DTYPE_FP8_E4M3)
            format = gg::kInE5M2xE4M3;
        else
            return fail(GG_ERR_INVALID, "unsupported pair of fp8 formats");
    } else if ((a_dtype != GG_DTYPE_BF16 && a_dtype != GG_DTYPE_FP16) || b_dtype != a_dtype) {
        return fail(GG_ERR_INVALID, "dtypes must be equal bf16 / fp16 types, or fp8 formats");
    }
    const int     layout   = op == GG_OP_FORWARD ? gg::kFwd : op == GG_OP_DGRAD ? gg::kDgrad : gg::kWgrad;
    // kernel terms (KernelArgs): output columns N_out, contraction K_c, output rows
    const int64_t n_out    = op == GG_OP_FORWARD ? n : k;
    const int64_t k_c      = op == GG_OP_FORWARD ? k : op == GG_OP_DGRAD ? n : 0; // wgrad: per group
    const int64_t out_rows = op == GG_OP_WGRAD ? int64_t(group_num) * n : total_m;
    const bool    has_output = out_rows > 0 && n_out > 0;
    const bool    reads      = op == GG_OP_WGRAD ? total_m > 0 : (total_m > 0 && k_c > 0);
    if (has_output && (out == nullptr || (reads && (a == nullptr || b == nullptr))))
        return fail(GG_ERR_INVALID, "the inputs and the output must be device pointers");
    if (f8 && has_output && reads && (a_scale == nullptr || b_scale == nullptr))
        return fail(GG_ERR_INVALID, "fp8 scales must be device pointers");
    // 16-byte rows; transposed fp8 operands move 16-column blocks
    const int64_t align_n = (f8 && op != GG_OP_FORWARD) ? 16 : 8;
    const int64_t align_k = f8 ? 16 : 8;
    if (n % align_n != 0)
        return fail(GG_ERR_UNSUPPORTED, "N must be a multiple of " + std::to_string(align_n));
    if (k % align_k != 0)
        return fail(GG_ERR_UNSUPPORTED, "K must be a multiple of " + std::to_string(align_k));
    if (has_output && (!aligned16(out) || (reads && (!aligned16(a) || !aligned16(b)))))
        return fail(GG_ERR_UNSUPPORTED, "buffers must be 16-byte aligned");
    if (k > (int64_t(1) << 21) || n > (int64_t(1) << 21))
        return fail(GG_ERR_UNSUPPORTED, "N and K must be at most 2097152");
    const int64_t lim   = int64_t(1) << 31;
    const int64_t es    = f8 ? 1 : 2;
    const int64_t steps = f8 ? 128 : gg::kTileK;
    if (op == GG_OP_DGRAD && (n + steps) * k * es >= lim)
        return fail(GG_ERR_UNSUPPORTED, "one group's w must be smaller than 2 GiB");
    // wgrad: a group may hold every row
    const int64_t wg_rows = std::max<int64_t>(total_m, gg::kCrossMinStepsHost * steps) + steps;
    if (op == GG_OP_WGRAD && (wg_rows * n * es >= lim || wg_rows * k * es >= lim))
        return fail(GG_ERR_UNSUPPORTED, "grad_out and x rows must be smaller than 2 GiB");
    const int64_t n_tiles = gg::cdiv(n_out, gg::kTileN);
    // wgrad: output tiles do not depend on the sizes, m_out rows per group
    const int64_t wgrad_tiles = op == GG_OP_WGRAD ? int64_t(group_num) * gg::cdiv(n, gg::kTileM) * n_tiles : 0;
    if (wgrad_tiles > INT32_MAX)
        return fail(GG_ERR_UNSUPPORTED, "too many tiles for 32-bit tile indices");

    plan->mode        = gg::make_mode(layout, format);
    plan->dtype       = f8 ? GG_DTYPE_BF16 : a_dtype; // output
    plan->group_num   = group_num;
    plan->n           = n_out;
    plan->k           = k_c;
    plan->total_m     = out_rows;
    plan->in_rows     = total_m;
    plan->x           = a;
    plan->w           = b;
    plan->out         = out;
    plan->device_lens = true;
    plan->d_lens      = group_lens;
    plan->d_offs      = group_offs;
    std::string what;
    if (!noalloc)
        what = std::string(op == GG_OP_FORWARD ? "" : op == GG_OP_DGRAD ? "dgrad " : "wgrad ") +
               (format == gg::kIn16     ? std::string(a_dtype == GG_DTYPE_BF16 ? "bf16" : "fp16")
                : format == gg::kInE4M3 ? std::string("fp8 e4m3")
                : format == gg::kInE5M2 ? std::string("fp8 e5m2")
                                        : std::string("fp8 e5m2 x e4m3"));
    const bool no_launch = !has_output || group_num == 0 || (op != GG_OP_WGRAD && k_c == 0);
    if (no_launch) {
        // forward / dgrad with an empty contraction: the run zero-fills the output
        if (!noalloc)
            plan->detail = "mi355x " + what + ": no launch (" +
                           (has_output && group_num > 0
                                ? (op == GG_OP_FORWARD ? "K = 0, zero fill" : "empty contraction, zero fill")
                                : "empty output") +
                           ")";
        if (!has_output || group_num == 0)
            plan->total_m = 0;
        return GG_OK;
    }
    int cus = 0, n_xcd = 1;
    const size_t table_bytes = static_cast<size_t>(group_num) * sizeof(gg::GroupEntry);
    if (noalloc) {
        NoAllocDevice d;
        if (const int st = noalloc_device(&d); st != GG_OK)
            return st;
        cus            = d.cus;
        n_xcd          = d.n_xcd;
        plan->d_groups = static_cast<gg::GroupEntry *>(d.scratch);
        plan->d_header = reinterpret_cast<gg::TableHeader *>(static_cast<char *>(d.scratch) + kNoAllocTableBytes);
    } else {
        hipDeviceProp_t prop;
        if (device_props(&prop) != GG_OK)
            return GG_ERR_HIP;
        cus   = prop.multiProcessorCount;
        n_xcd = xcd_count(prop);
        // Table + header in one allocation; the header is written by every run.
        const hipError_t e = hipMalloc(&plan->d_groups, table_bytes + sizeof(gg::TableHeader));
        if (e != hipSuccess) {
            plan->d_groups = nullptr;
            return hip_fail(e, "group table allocation");
        }
        plan->d_header = reinterpret_cast<gg::TableHeader *>(reinterpret_cast<char *>(plan->d_groups) +
                                                             table_bytes);
    }
    fill_args(plan, 1);
    gg::KernelArgs &ka = plan->args;
    ka.k_tiles         = op == GG_OP_WGRAD ? 1 : static_cast<int>(gg::cdiv(k_c, steps));
    // tails (see KernelArgs): forward has K-major operands only; dgrad's w columns are the k of
    // its output; wgrad's K steps depend on the device-resident sizes, so it keeps the masks
    ka.tails = op == GG_OP_FORWARD ? (k_c % steps != 0)
               : op == GG_OP_DGRAD ? (k_c % steps != 0 || k % gg::kTileN != 0)
                                   : 1;
    ka.x_scale         = f8 ? a_scale : nullptr;
    ka.w_scale         = f8 ? b_scale : nullptr;
    if (op != GG_OP_FORWARD) {
        ka.lda = static_cast<int>(n);
        ka.ldb = static_cast<int>(k);
    }
    if (op == GG_OP_WGRAD) {
        // The K-step counts depend on the sizes; a cross-tile wgrad tile runs at least
        // kCrossMinStepsHost of them (zeros past its group's rows), so the cross-tile variant runs.
        ka.m_out          = static_cast<int>(n);
        ka.min_steps      = gg::kCrossMinStepsHost;
        plan->total_tiles = static_cast<int>(wgrad_tiles);
        plan->grid        = static_cast<int>(std::min<int64_t>(cus, wgrad_tiles));
        ka.total_tiles    = plan->total_tiles;
        ka.d_total        = nullptr;
    } else {
        // Tile count is unknown here: one workgroup per CU, or fewer if even the largest routing
        // (every group's rows tiled separately) has fewer tiles.
        const int64_t max_tiles = (gg::cdiv(total_m, gg::kTileM) + group_num) * n_tiles;
        plan->grid     = static_cast<int>(std::min<int64_t>(cus, max_tiles));
        ka.total_tiles = 0;
        ka.d_total     = &plan->d_header->total_tiles;
    }
    // At most kInKernelTableGroups groups: the GEMM builds the table itself (one group per lane of
    // every wave) and writes the header, so a run is one launch. Not for an fp8 wgrad plan that
    // would run the per-tile variant (only in builds without the cross-tile pipeline): that
    // instance has no in-kernel table.
    gg::KernelArgs probe = ka;
    probe.d_lens         = group_lens;
    const bool lane_table_ok = !(f8 && op == GG_OP_WGRAD && !gg::uses_cross_tile(probe, plan->grid, plan->mode));
    if (group_num <= gg::kInKernelTableGroups && lane_table_ok) {
        plan->in_kernel_table = true;
        ka.d_lens             = group_lens;
        ka.d_offs             = group_offs;
        ka.lens_rows          = total_m;
        ka.d_header           = plan->d_header;
        ka.d_total            = nullptr;
    }
    ka.n_xcd = plan->grid % n_xcd == 0 ? n_xcd : 1;
    if (!noalloc)
        plan->detail = "mi355x " + what + " persistent 256x256x" + std::to_string(f8 ? 128 : 64) + " grid=" +
                       std::to_string(plan->grid) + " tiles=" +
                       (op == GG_OP_WGRAD ? std::to_string(plan->total_tiles) : std::string("device")) +
                       " xcd=" + std::to_string(ka.n_xcd) +
                       (gg::uses_cross_tile(ka, plan->grid, plan->mode) ? " cross-tile" : " per-tile") +
                       (ka.band != gg::kBand ? " band=" + std::to_string(ka.band) : "") +
                       (plan->in_kernel_table ? " (device group sizes, in-kernel table)" : " (device group sizes)");
    return GG_OK;
}

// Enqueue a plan's launches on `stream` (gg_run). zero_kernel: an empty contraction zero-fills
// the output with a fill kernel instead of hipMemsetAsync (which a captured graph must not
// hold).
int run_plan(const gg_plan *plan, void *stream, bool zero_kernel) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (plan->device_lens && plan->d_groups != nullptr) {
        hipError_t e = hipSuccess;
        if (!plan->in_kernel_table) {
            e = gg::launch_build_group_table(plan->d_lens, plan->d_offs, plan->group_num, plan->in_rows,
                                             plan->args.n_tiles, plan->d_groups, plan->d_header, s,
                                             plan->args.m_out);
            if (e != hipSuccess)
                return hip_fail(e, "group table launch");
        }
        e = gg::launch_grouped_gemm(plan->args, plan->dtype == GG_DTYPE_FP16, plan->grid, s, plan->mode);
        if (e != hipSuccess)
            return hip_fail(e, "grouped GEMM launch");
        return GG_OK;
    }
    if (plan->total_tiles == 0) {
        // K == 0 with a non-empty output: out = 0.
        if (plan->total_m > 0 && plan->n > 0 && plan->k == 0) {
            const size_t     bytes = size_t(plan->total_m) * plan->n * 2;
            const hipError_t e     = zero_kernel ? gg::launch_zero_fill(plan->out, bytes, s)
                                                 : hipMemsetAsync(plan->out, 0, bytes, s);
            if (e != hipSuccess)
                return hip_fail(e, zero_kernel ? "zero fill launch" : "hipMemsetAsync");
        }
        return GG_OK;
    }
    if (plan->small) {
        const hipError_t e = gg::launch_small_gemm(plan->sargs, plan->dtype == GG_DTYPE_FP16, s);
        return e == hipSuccess ? GG_OK : hip_fail(e, "small-tile GEMM launch");
    }
    hipError_t e = gg::launch_grouped_gemm(plan->args, plan->dtype == GG_DTYPE_FP16, plan->grid, s, plan->mode);
    if (e != hipSuccess)
        return hip_fail(e, "grouped GEMM launch");
    if (plan->args.splits > 1) {
        e = gg::launch_split_reduce(plan->args, plan->dtype == GG_DTYPE_FP16, s, plan->mode);
        if (e != hipSuccess)
            return hip_fail(e, "split-K reduction launch");
    }
    if (plan->args.tail_splits > 1) {
        e = gg::launch_tail_reduce(plan->args, plan->dtype == GG_DTYPE_FP16, plan->grid, s);
        if (e != hipSuccess)
            return hip_fail(e, "tail-split reduction launch");
    }
    return GG_OK;
}

} // namespace

extern "C" {

int gg_prepare(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
               const void *x, const void *w, void *out, void *stream, gg_plan **plan_out) {
    g_last_error.clear();
    if (plan_out == nullptr)
        return fail(GG_ERR_INVALID, "plan_out is null");
    *plan_out = nullptr;
    if (group_num > 0 && group_m == nullptr)
        return fail(GG_ERR_INVALID, "group_m is null");

    int64_t total_m = 0;
    for (int g = 0; g < group_num; ++g) {
        if (group_m[g] < 0)
            return fail(GG_ERR_INVALID, "group_m[" + std::to_string(g) + "] < 0");
        total_m += group_m[g];
    }
    const bool has_output = total_m > 0 && n > 0;
    const int  st         = check_problem(dtype, group_num, n, k, has_output, x, w, out);
    if (st != GG_OK)
        return st;

    auto *plan = new (std::nothrow) gg_plan;
    if (plan == nullptr)
        return fail(GG_ERR_INVALID, "out of host memory");
    plan->dtype     = dtype;
    plan->group_num = group_num;
    plan->n         = n;
    plan->k         = k;
    plan->total_m   = total_m;
    plan->x         = x;
    plan->w         = w;
    plan->out       = out;

    // Group table: row offset, rows and first tile of every group (empty groups own no
    // tiles; the kernel steps over them while scanning forward).
    const int64_t n_tiles = gg::cdiv(n, gg::kTileN);
    std::vector<gg::GroupEntry> table(static_cast<size_t>(group_num));
    const int64_t tiles = gg::build_group_table(group_m, group_num, n_tiles, table.data());
    if (tiles < 0) {
        delete plan;
        return fail(GG_ERR_UNSUPPORTED, "too many rows or tiles for 32-bit tile indices");
    }
    plan->total_tiles = has_output && k > 0 ? static_cast<int>(tiles) : 0;

    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (plan->total_tiles > 0) {
        hipDeviceProp_t prop;
        if (device_props(&prop) != GG_OK) {
            delete plan;
            return GG_ERR_HIP;
        }
        const size_t bytes = table.size() * sizeof(gg::GroupEntry);
        hipError_t   e     = hipMalloc(&plan->d_groups, bytes);
        if (e == hipSuccess)
            e = hipMemcpyAsync(plan->d_groups, table.data(), bytes, hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            if (plan->d_groups != nullptr)
                (void)hipFree(plan->d_groups);
            delete plan;
            return hip_fail(e, "group table upload");
        }
        // Persistent grid: one workgroup per CU (160 KB of LDS each), never more than tiles.
        plan->grid = std::min(prop.multiProcessorCount, plan->total_tiles);
        fill_args(plan, xcd_count(prop));
        gg::KernelArgs &a = plan->args;
        a.total_tiles     = plan->total_tiles;
        a.d_total         = nullptr;
        a.tails           = k % gg::kTileK != 0; // K-major operands: only a partial K step
        if (setup_split_k(plan, prop) != GG_OK) {
            free_plan(plan);
            return GG_ERR_HIP;
        }
        if (const int st2 = use_short_tiles(plan, group_m, s); st2 != GG_OK) {
            free_plan(plan);
            return st2;
        }
        if (use_short_wide_tiles(plan, group_m, prop, s) != GG_OK) {
            free_plan(plan);
            return GG_ERR_HIP;
        }
        if (use_narrow_tiles(plan, group_m, prop, s) != GG_OK) {
            free_plan(plan);
            return GG_ERR_HIP;
        }
        if (setup_tail_split(plan) != GG_OK) {
            free_plan(plan);
            return GG_ERR_HIP;
        }
        if (const int st3 = setup_tile_desc(plan, group_m, s); st3 != GG_OK) {
            free_plan(plan);
            return st3;
        }
        if (const int st4 = use_small_tiles(plan, group_m, prop, s); st4 != GG_OK) {
            free_plan(plan);
            return st4;
        }
        const std::string dt = dtype == GG_DTYPE_BF16 ? "bf16" : "fp16";
        if (plan->small)
            plan->detail = "mi355x small 128x128x64 " + dt + " grid=" + std::to_string(plan->grid) +
                           " tiles=" + std::to_string(plan->total_tiles) +
                           (plan->sargs.stages == gg::kSmallStagesTwo ? " two-per-cu" : "") +
                           (plan->sargs.splits > 1 ? " split-k=" + std::to_string(plan->sargs.splits) : "");
        else
            plan->detail = "mi355x persistent " + std::to_string(a.tile_m) + "x" + std::to_string(a.tile_n) +
                           "x64 " + dt + " grid=" + std::to_string(plan->grid) +
                           " tiles=" + std::to_string(plan->total_tiles) + " xcd=" + std::to_string(a.n_xcd) +
                           (gg::uses_cross_tile(a, plan->grid) ? " cross-tile" : " per-tile") +
                           (a.band != gg::kBand ? " band=" + std::to_string(a.band) : "") +
                           (a.splits > 1 ? " split-k=" + std::to_string(a.splits) : "") +
                           (a.tail_splits > 1 ? " tail-split=" + std::to_string(a.tail_splits) : "");
    } else {
        plan->detail = "mi355x: no launch (" +
                       std::string(has_output ? "K = 0, zero fill" : "empty output") + ")";
    }
    *plan_out = plan;
    return GG_OK;
}

// Backward plans in kernel terms (see KernelArgs): out (rows x N) = A B^T per group with the
// contraction K. dgrad: A = grad_out (K-major, row stride n), B^T = w[g] stored n x k,
// N = k, K = n. wgrad: A^T = grad_out rows of the group (row stride n), B^T = x rows (row stride
// k), out = grad_w[g] n x k, N = k, K = the group's rows.
// dtype_a / dtype_b: formats of grad_out and of the other operand. 16-bit: both the same, no
// scales. fp8: e4m3 x e4m3, e5m2 x e5m2 or e5m2 gradient x e4m3, bf16 out scaled by a_scale[0] *
// b_scale[g].
static int prepare_backward(int layout, int dtype_a, int dtype_b, int group_num, int64_t n, int64_t k,
                            const int64_t *group_m, const void *a, const void *b, const float *a_scale,
                            const float *b_scale, void *out, void *stream, gg_plan **plan_out) {
    g_last_error.clear();
    if (plan_out == nullptr)
        return fail(GG_ERR_INVALID, "plan_out is null");
    *plan_out = nullptr;
    if (group_num > 0 && group_m == nullptr)
        return fail(GG_ERR_INVALID, "group_m is null");
    const bool f8     = dtype_a == GG_DTYPE_FP8_E4M3 || dtype_a == GG_DTYPE_FP8_E5M2;
    int        format = gg::kIn16;
    if (f8) {
        if (dtype_a == GG_DTYPE_FP8_E4M3 && dtype_b == GG_DTYPE_FP8_E4M3)
            format = gg::kInE4M3;
        else if (dtype_a == GG_DTYPE_FP8_E5M2 && dtype_b == GG_DTYPE_FP8_E5M2)
            format = gg::kInE5M2;
        else if (dtype_a == GG_DTYPE_FP8_E5M2 && dtype_b == GG_DTYPE_FP8_E4M3)
            format = gg::kInE5M2xE4M3;
        else
            return fail(GG_ERR_INVALID, "fp8 formats must be e4m3 x e4m3, e5m2 x e5m2 or e5m2 gradient x e4m3");
    } else if ((dtype_a != GG_DTYPE_BF16 && dtype_a != GG_DTYPE_FP16) || dtype_b != dtype_a) {
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_BF16 or GG_DTYPE_FP16");
    }
    int64_t total_m = 0, max_m = 0;
    for (int g = 0; g < group_num; ++g) {
        if (group_m[g] < 0)
            return fail(GG_ERR_INVALID, "group_m[" + std::to_string(g) + "] < 0");
        total_m += group_m[g];
        max_m = std::max(max_m, group_m[g]);
    }
    const bool dgrad = layout == gg::kDgrad;
    // Output rows: grad_x has total_m, grad_w has group_num * n.
    const int64_t out_rows   = dgrad ? total_m : int64_t(group_num) * n;
    const bool    has_output = out_rows > 0 && k > 0;
    // Both operands are read when the contraction (n for dgrad, the rows for wgrad) is non-zero.
    const bool reads = dgrad ? (total_m > 0 && n > 0) : (total_m > 0);
    if (group_num < 0 || n < 0 || k < 0)
        return fail(GG_ERR_INVALID, "group_num, n and k must be >= 0");
    if (has_output && (out == nullptr || (reads && (a == nullptr || b == nullptr))))
        return fail(GG_ERR_INVALID, "grad_out, the second operand and the output must be device pointers");
    if (f8 && has_output && reads && (a_scale == nullptr || b_scale == nullptr))
        return fail(GG_ERR_INVALID, "fp8 scales must be device pointers");
    // 16-byte rows; fp8 transposed operands move 16-column blocks
    const int64_t align = f8 ? 16 : 8;
    if (n % align != 0)
        return fail(GG_ERR_UNSUPPORTED, std::string("N must be a multiple of ") + std::to_string(align));
    if (k % align != 0)
        return fail(GG_ERR_UNSUPPORTED, std::string("K must be a multiple of ") + std::to_string(align));
    if (has_output && (!aligned16(out) || (reads && (!aligned16(a) || !aligned16(b)))))
        return fail(GG_ERR_UNSUPPORTED, "buffers must be 16-byte aligned");
    if (k > (int64_t(1) << 21) || n > (int64_t(1) << 21))
        return fail(GG_ERR_UNSUPPORTED, "N and K must be at most 2097152");
    // 32-bit byte offsets inside one group's transposed operand, including the rows a partial
    // last K step addresses past the end (up to one step more).
    const int64_t lim   = int64_t(1) << 31;
    const int64_t es    = f8 ? 1 : 2;
    const int64_t steps = f8 ? 128 : gg::kTileK; // contraction rows per K step
    if (dgrad && (n + steps) * k * es >= lim)
        return fail(GG_ERR_UNSUPPORTED, "one group's w must be smaller than 2 GiB");
    // (wgrad: a short group's tile addresses kCrossMinStepsHost steps)
    const int64_t rows_addr = std::max<int64_t>(max_m, gg::kCrossMinStepsHost * steps) + steps;
    if (!dgrad && (rows_addr * n * es >= lim || rows_addr * k * es >= lim))
        return fail(GG_ERR_UNSUPPORTED, "one group's rows of grad_out and x must be smaller than 2 GiB");

    auto *plan = new (std::nothrow) gg_plan;
    if (plan == nullptr)
        return fail(GG_ERR_INVALID, "out of host memory");
    plan->mode      = gg::make_mode(layout, format);
    plan->dtype     = f8 ? GG_DTYPE_BF16 : dtype_a; // output
    plan->group_num = group_num;
    plan->n         = k;                      // output columns
    plan->k         = dgrad ? n : 0;          // contraction (wgrad: per group)
    plan->total_m   = out_rows;               // rows zeroed when there is nothing to read
    plan->x         = a;
    plan->w         = b;
    plan->out       = out;

    const int64_t n_tiles = gg::cdiv(k, gg::kTileN);
    std::vector<gg::GroupEntry> table(static_cast<size_t>(group_num));
    const int64_t tiles = gg::build_group_table(group_m, group_num, n_tiles, table.data(), dgrad ? 0 : n);
    if (tiles < 0) {
        delete plan;
        return fail(GG_ERR_UNSUPPORTED, "too many rows or tiles for 32-bit tile indices");
    }
    // dgrad with n == 0: grad_x = 0 (gg_run zero-fills). wgrad with no rows: the tiles run and
    // store zeros (each group's K steps read nothing).
    plan->total_tiles = has_output && (!dgrad || n > 0) ? static_cast<int>(tiles) : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const std::string what = std::string(dgrad ? "dgrad" : "wgrad") +
                             (format == gg::kIn16         ? ""
                              : format == gg::kInE4M3     ? " fp8 e4m3"
                              : format == gg::kInE5M2     ? " fp8 e5m2"
                                                          : " fp8 e5m2 x e4m3");
    if (plan->total_tiles > 0) {
        hipDeviceProp_t prop;
        if (device_props(&prop) != GG_OK) {
            delete plan;
            return GG_ERR_HIP;
        }
        const size_t bytes = table.size() * sizeof(gg::GroupEntry);
        hipError_t   e     = hipMalloc(&plan->d_groups, bytes);
        if (e == hipSuccess)
            e = hipMemcpyAsync(plan->d_groups, table.data(), bytes, hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            if (plan->d_groups != nullptr)
                (void)hipFree(plan->d_groups);
            delete plan;
            return hip_fail(e, "group table upload");
        }
        plan->grid = std::min(prop.multiProcessorCount, plan->total_tiles);
        fill_args(plan, xcd_count(prop));
        gg::KernelArgs &ka = plan->args;
        ka.total_tiles     = plan->total_tiles;
        ka.d_total         = nullptr;
        ka.lda             = static_cast<int>(n);
        ka.ldb             = static_cast<int>(k);
        ka.m_out           = dgrad ? 0 : static_cast<int>(n);
        ka.k_tiles         = dgrad ? static_cast<int>(gg::cdiv(n, steps)) : 1;
        if (!dgrad) // fewest K steps of a tile: a cross-tile wgrad tile runs at least
                    // kCrossMinStepsHost (zeros past a short or empty group's rows)
            ka.min_steps = gg::kCrossMinStepsHost;
        ka.x_scale         = f8 ? a_scale : nullptr;
        ka.w_scale         = f8 ? b_scale : nullptr;
        // tails (see KernelArgs). dgrad: the contraction n and w's columns k. wgrad: every group's
        // rows (its contraction) and the columns of grad_out (n) and x (k).
        if (dgrad) {
            ka.tails = n % steps != 0 || k % gg::kTileN != 0;
        } else { // and the zero steps of a group shorter than kCrossMinStepsHost steps
            bool t = n % gg::kTileN != 0 || k % gg::kTileN != 0;
            for (int g = 0; g < group_num; ++g)
                t = t || group_m[g] % steps != 0 || group_m[g] < gg::kCrossMinStepsHost * steps;
            ka.tails = t;
        }
        // wgrad's K steps differ per group: no split
        if (dgrad && setup_split_k(plan, prop) != GG_OK) {
            free_plan(plan);
            return GG_ERR_HIP;
        }
        if (dgrad && !f8) { // short tiles: the output rows are the groups' tokens
            if (const int st2 = use_short_tiles(plan, group_m, s); st2 != GG_OK) {
                free_plan(plan);
                return st2;
            }
        }
        if (const int st3 = setup_tile_desc(plan, group_m, s); st3 != GG_OK) {
            free_plan(plan);
            return st3;
        }

        plan->detail = "mi355x " + what + " persistent " + std::to_string(ka.tile_m) + "x256x" +
                       std::to_string(f8 ? 128 : 64) + " " +
                       (f8 ? "bf16-out" : dtype_a == GG_DTYPE_BF16 ? "bf16" : "fp16") +
                       " grid=" + std::to_string(plan->grid) + " tiles=" + std::to_string(plan->total_tiles) +
                       " xcd=" + std::to_string(ka.n_xcd) +
                       (gg::uses_cross_tile(ka, plan->grid, plan->mode) ? " cross-tile" : " per-tile") +
                       (ka.band != gg::kBand ? " band=" + std::to_string(ka.band) : "") +
                       (ka.splits > 1 ? " split-k=" + std::to_string(ka.splits) : "") +
                       (ka.tail_splits > 1 ? " tail-split=" + std::to_string(ka.tail_splits) : "");
    } else {
        plan->detail = "mi355x " + what + ": no launch (" +
                       (has_output ? "empty contraction, zero fill" : "empty output") + ")";
        if (!has_output)
            plan->total_m = 0;
    }
    *plan_out = plan;
    return GG_OK;
}

int gg_prepare_fp8(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                   const void *x, const void *w, const float *x_scale, const float *w_scale, void *out,
                   void *stream, gg_plan **plan_out) {
    g_last_error.clear();
    if (plan_out == nullptr)
        return fail(GG_ERR_INVALID, "plan_out is null");
    *plan_out = nullptr;
    if (dtype != GG_DTYPE_FP8_E4M3 && dtype != GG_DTYPE_FP8_E5M2)
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_FP8_E4M3 or GG_DTYPE_FP8_E5M2");
    if (group_num > 0 && group_m == nullptr)
        return fail(GG_ERR_INVALID, "group_m is null");
    int64_t total_m = 0;
    for (int g = 0; g < group_num; ++g) {
        if (group_m[g] < 0)
            return fail(GG_ERR_INVALID, "group_m[" + std::to_string(g) + "] < 0");
        total_m += group_m[g];
    }
    if (group_num < 0 || n < 0 || k < 0)
        return fail(GG_ERR_INVALID, "group_num, n and k must be >= 0");
    const bool has_output = total_m > 0 && n > 0;
    if (has_output && (out == nullptr || (k > 0 && (x == nullptr || w == nullptr || x_scale == nullptr ||
                                                    w_scale == nullptr))))
        return fail(GG_ERR_INVALID, "x, w, the scales and out must be device pointers");
    if (n % 8 != 0)
        return fail(GG_ERR_UNSUPPORTED, "N must be a multiple of 8 (16-byte output rows)");
    if (k % 16 != 0)
        return fail(GG_ERR_UNSUPPORTED, "K must be a multiple of 16 for fp8 (16-byte input rows)");
    if (has_output && (!aligned16(out) || (k > 0 && (!aligned16(x) || !aligned16(w)))))
        return fail(GG_ERR_UNSUPPORTED, "x, w and out must be 16-byte aligned");
    if (k > (int64_t(1) << 21) || n > (int64_t(1) << 21))
        return fail(GG_ERR_UNSUPPORTED, "N and K must be at most 2097152");

    auto *plan = new (std::nothrow) gg_plan;
    if (plan == nullptr)
        return fail(GG_ERR_INVALID, "out of host memory");
    plan->mode      = gg::make_mode(gg::kFwd, dtype == GG_DTYPE_FP8_E4M3 ? gg::kInE4M3 : gg::kInE5M2);
    plan->dtype     = GG_DTYPE_BF16; // output
    plan->group_num = group_num;
    plan->n         = n;
    plan->k         = k;
    plan->total_m   = total_m;
    plan->x         = x;
    plan->w         = w;
    plan->out       = out;
    const int64_t n_tiles = gg::cdiv(n, gg::kTileN);
    std::vector<gg::GroupEntry> table(static_cast<size_t>(group_num));
    const int64_t tiles = gg::build_group_table(group_m, group_num, n_tiles, table.data());
    if (tiles < 0) {
        delete plan;
        return fail(GG_ERR_UNSUPPORTED, "too many rows or tiles for 32-bit tile indices");
    }
    plan->total_tiles = has_output && k > 0 ? static_cast<int>(tiles) : 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (plan->total_tiles > 0) {
        hipDeviceProp_t prop;
        if (device_props(&prop) != GG_OK) {
            delete plan;
            return GG_ERR_HIP;
        }
        const size_t bytes = table.size() * sizeof(gg::GroupEntry);
        hipError_t   e     = hipMalloc(&plan->d_groups, bytes);
        if (e == hipSuccess)
            e = hipMemcpyAsync(plan->d_groups, table.data(), bytes, hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            if (plan->d_groups != nullptr)
                (void)hipFree(plan->d_groups);
            delete plan;
            return hip_fail(e, "group table upload");
        }
        plan->grid = std::min(prop.multiProcessorCount, plan->total_tiles);
        fill_args(plan, xcd_count(prop));
        gg::KernelArgs &a = plan->args;
        a.total_tiles     = plan->total_tiles;
        a.d_total         = nullptr;
        a.k_tiles         = static_cast<int>(gg::cdiv(k, 128)); // 128 fp8 values per K step
        a.tails           = k % 128 != 0;
        a.x_scale         = x_scale;
        a.w_scale         = w_scale;
        if (setup_split_k(plan, prop) != GG_OK) {
            free_plan(plan);
            return GG_ERR_HIP;
        }
        if (const int st3 = setup_tile_desc(plan, group_m, s); st3 != GG_OK) {
            free_plan(plan);
            return st3;
        }
        plan->detail = std::string("mi355x fp8 ") + (dtype == GG_DTYPE_FP8_E4M3 ? "e4m3" : "e5m2") +
                       " persistent 256x256x128 bf16-out grid=" + std::to_string(plan->grid) +
                       " tiles=" + std::to_string(plan->total_tiles) + " xcd=" + std::to_string(a.n_xcd) +
                       (gg::uses_cross_tile(a, plan->grid, plan->mode) ? " cross-tile" : " per-tile") +
                       (a.band != gg::kBand ? " band=" + std::to_string(a.band) : "") +
                       (a.splits > 1 ? " split-k=" + std::to_string(a.splits) : "") +
                       (a.tail_splits > 1 ? " tail-split=" + std::to_string(a.tail_splits) : "");
    } else {
        plan->detail = std::string("mi355x fp8: no launch (") +
                       (has_output ? "K = 0, zero fill" : "empty output") + ")";
    }
    *plan_out = plan;
    return GG_OK;
}

int gg_prepare_dgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                     const void *grad_out, const void *w, void *grad_x, void *stream, gg_plan **plan_out) {
    if (dtype != GG_DTYPE_BF16 && dtype != GG_DTYPE_FP16)
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_BF16 or GG_DTYPE_FP16");
    return prepare_backward(gg::kDgrad, dtype, dtype, group_num, n, k, group_m, grad_out, w, nullptr, nullptr,
                            grad_x, stream, plan_out);
}

int gg_prepare_wgrad(int dtype, int group_num, int64_t n, int64_t k, const int64_t *group_m,
                     const void *grad_out, const void *x, void *grad_w, void *stream, gg_plan **plan_out) {
    if (dtype != GG_DTYPE_BF16 && dtype != GG_DTYPE_FP16)
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_BF16 or GG_DTYPE_FP16");
    return prepare_backward(gg::kWgrad, dtype, dtype, group_num, n, k, group_m, grad_out, x, nullptr, nullptr,
                            grad_w, stream, plan_out);
}

int gg_prepare_dgrad_fp8(int grad_dtype, int w_dtype, int group_num, int64_t n, int64_t k,
                         const int64_t *group_m, const void *grad_out, const void *w, const float *grad_scale,
                         const float *w_scale, void *grad_x, void *stream, gg_plan **plan_out) {
    if (grad_dtype != GG_DTYPE_FP8_E4M3 && grad_dtype != GG_DTYPE_FP8_E5M2)
        return fail(GG_ERR_INVALID, "grad_dtype must be GG_DTYPE_FP8_E4M3 or GG_DTYPE_FP8_E5M2");
    return prepare_backward(gg::kDgrad, grad_dtype, w_dtype, group_num, n, k, group_m, grad_out, w, grad_scale,
                            w_scale, grad_x, stream, plan_out);
}

int gg_prepare_wgrad_fp8(int grad_dtype, int x_dtype, int group_num, int64_t n, int64_t k,
                         const int64_t *group_m, const void *grad_out, const void *x, const float *grad_scale,
                         const float *x_scale, void *grad_w, void *stream, gg_plan **plan_out) {
    if (grad_dtype != GG_DTYPE_FP8_E4M3 && grad_dtype != GG_DTYPE_FP8_E5M2)
        return fail(GG_ERR_INVALID, "grad_dtype must be GG_DTYPE_FP8_E4M3 or GG_DTYPE_FP8_E5M2");
    return prepare_backward(gg::kWgrad, grad_dtype, x_dtype, group_num, n, k, group_m, grad_out, x, grad_scale,
                            x_scale, grad_w, stream, plan_out);
}

int gg_prepare_device_lens(int dtype, int group_num, int64_t total_m, int64_t n, int64_t k,
                           const int64_t *group_lens, const int64_t *group_offs, const void *x,
                           const void *w, void *out, void *stream, gg_plan **plan_out) {
    if (dtype != GG_DTYPE_BF16 && dtype != GG_DTYPE_FP16) {
        g_last_error.clear();
        if (plan_out != nullptr)
            *plan_out = nullptr;
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_BF16 or GG_DTYPE_FP16");
    }
    return gg_prepare_device_lens_op(GG_OP_FORWARD, dtype, dtype, group_num, total_m, n, k, group_lens,
                                     group_offs, x, w, nullptr, nullptr, out, stream, plan_out);
}

int gg_prepare_device_lens_op(int op, int a_dtype, int b_dtype, int group_num, int64_t total_m, int64_t n,
                              int64_t k, const int64_t *group_lens, const int64_t *group_offs, const void *a,
                              const void *b, const float *a_scale, const float *b_scale, void *out,
                              void *stream, gg_plan **plan_out) {
    (void)stream;
    g_last_error.clear();
    if (plan_out == nullptr)
        return fail(GG_ERR_INVALID, "plan_out is null");
    *plan_out = nullptr;
    auto *plan = new (std::nothrow) gg_plan;
    if (plan == nullptr)
        return fail(GG_ERR_INVALID, "out of host memory");
    const int st = plan_device_lens(plan, false, op, a_dtype, b_dtype, group_num, total_m, n, k, group_lens,
                                    group_offs, a, b, a_scale, b_scale, out);
    if (st != GG_OK) {
        free_plan(plan);
        return st;
    }
    *plan_out = plan;
    return GG_OK;
}

int gg_run_device_lens_noalloc(int op, int a_dtype, int b_dtype, int group_num, int64_t total_m, int64_t n,
                               int64_t k, const int64_t *group_lens, const int64_t *group_offs, const void *a,
                               const void *b, const float *a_scale, const float *b_scale, void *out,
                               void *stream) {
    g_last_error.clear();
    if (group_num > kNoAllocMaxGroups)
        return fail(GG_ERR_UNSUPPORTED, "gg_run_device_lens_noalloc takes at most " +
                                            std::to_string(kNoAllocMaxGroups) + " groups (got " +
                                            std::to_string(group_num) + ")");
    gg_plan plan; // on the stack: its table is the device's scratch array
    const int st = plan_device_lens(&plan, true, op, a_dtype, b_dtype, group_num, total_m, n, k, group_lens,
                                    group_offs, a, b, a_scale, b_scale, out);
    if (st != GG_OK)
        return st;
    return run_plan(&plan, stream, true);
}

int gg_run(const gg_plan *plan, void *stream) {
    if (plan == nullptr)
        return fail(GG_ERR_INVALID, "plan is null");
    return run_plan(plan, stream, false);
}

void gg_release(gg_plan *plan) {
    if (plan == nullptr)
        return;
    free_plan(plan);
}

const char *gg_plan_detail(const gg_plan *plan) { return plan ? plan->detail.c_str() : ""; }

int gg_plan_grid(const gg_plan *plan) { return plan ? plan->grid : 0; }

int gg_plan_tiles(const gg_plan *plan) { return plan ? plan->total_tiles : 0; }

int gg_plan_device_status(const gg_plan *plan, void *stream, int *total_tiles) {
    g_last_error.clear();
    if (plan == nullptr)
        return fail(GG_ERR_INVALID, "plan is null");
    if (!plan->device_lens || plan->d_header == nullptr) {
        if (total_tiles != nullptr)
            *total_tiles = plan->total_tiles;
        return GG_OK;
    }
    gg::TableHeader h{};
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(&h, plan->d_header, sizeof(h), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e != hipSuccess)
        return hip_fail(e, "device status read");
    if (total_tiles != nullptr)
        *total_tiles = h.total_tiles;
    if (h.overflow != 0)
        return fail(GG_ERR_INVALID, "device group sizes: more than 2^31 tiles, nothing computed");
    if (h.first_bad >= 0)
        return fail(GG_ERR_INVALID, "device group sizes: group " + std::to_string(h.first_bad) +
                                        " has a negative length or rows outside [0, total_m); "
                                        "its rows were not written");
    return GG_OK;
}

int gg_compute_group_offs(const int64_t *group_lens, int64_t *group_offs, int group_num,
                          void *stream) {
    g_last_error.clear();
    if (group_num < 0)
        return fail(GG_ERR_INVALID, "group_num must be >= 0");
    if (group_offs == nullptr || (group_num > 0 && group_lens == nullptr))
        return fail(GG_ERR_INVALID, "group_lens and group_offs must be device pointers");
    const hipError_t e =
        gg::launch_group_offsets(group_lens, group_offs, group_num, static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return hip_fail(e, "group offsets launch");
    return GG_OK;
}

const char *gg_last_error(void) { return g_last_error.c_str(); }

int gg_fill_randn(int dtype, void *p, size_t count, uint64_t seed, void *stream) {
    g_last_error.clear();
    if (dtype != GG_DTYPE_BF16 && dtype != GG_DTYPE_FP16)
        return fail(GG_ERR_INVALID, "dtype must be GG_DTYPE_BF16 or GG_DTYPE_FP16");
    if (count > 0 && p == nullptr)
        return fail(GG_ERR_INVALID, "p is null");
    const hipError_t e = gg::launch_fill_randn(p, count, seed, dtype == GG_DTYPE_FP16,
                                               static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return hip_fail(e, "fill launch");
    return GG_OK;
}

int gg_clock_probe(uint64_t *dev_out, double seconds, void *stream) {
    g_last_error.clear();
    if (dev_out == nullptr)
        return fail(GG_ERR_INVALID, "dev_out is null");
    if (!(seconds > 0.0 && seconds <= 10.0))
        return fail(GG_ERR_INVALID, "seconds must be in (0, 10]");
    int        dev = 0, khz = 0;
    hipError_t e   = hipGetDevice(&dev);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess)
        return hip_fail(e, "wall clock rate");
    if (khz <= 0)
        return fail(GG_ERR_UNSUPPORTED, "the device reports no wall clock rate");
    const unsigned long long hz    = static_cast<unsigned long long>(khz) * 1000ull;
    const unsigned long long ticks = static_cast<unsigned long long>(seconds * static_cast<double>(hz));
    e = gg::launch_clock_probe(reinterpret_cast<unsigned long long *>(dev_out), ticks, hz,
                               static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return hip_fail(e, "clock probe launch");
    return GG_OK;
}

} // extern "C"
