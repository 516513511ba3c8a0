// Launch interface between the C ABI layer (gg_capi.hip) and the gfx950 kernel
// (gg_kernel.hip). Host-only declarations; no device code here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gg_schedule.h"

namespace gg {

// Kernel modes: an operand layout plus an input format, mode = layout + 4 * format.
enum Layout : int { kFwd = 0, kDgrad = 1, kWgrad = 2 };
enum InFormat : int {
    kIn16        = 0, // bf16 or fp16 inputs and output
    kInE4M3      = 1, // fp8 e4m3 A and B, bf16 output
    kInE5M2      = 2, // fp8 e5m2 A and B, bf16 output
    kInE5M2xE4M3 = 3  // fp8 e5m2 A (the gradient), e4m3 B, bf16 output
};
constexpr int make_mode(int layout, int format) { return layout + 4 * format; }

// Header of a device-built group table (follows the group_num entries).
struct TableHeader {
    int total_tiles; // tiles over all groups (0 if the count overflowed)
    int first_bad;   // first group whose length or offset was out of range, -1 if none
    int overflow;    // 1 if the tile count exceeded 32 bits (nothing is computed then)
    int reserved;
};

// Device-resident group sizes of at most this many groups: the grouped GEMM builds the group
// table itself (one group per lane of every wave), with no separate table launch.
constexpr int kInKernelTableGroups = 64;

// Kernel arguments, passed by value in the kernarg segment. Everything a workgroup needs
// to find its tiles: the device group table plus the problem-wide sizes.
// Kernel terms: out (rows x N) = A (rows x K) B^T (N x K) per group, K the contraction.
//   forward: A = x [sum(M), K], B = w [B, N, K], out [sum(M), N]
//   dgrad:   A = grad_out [sum(M), K], B^T = w[g] [K, N] (stored K x N), out = grad_x [sum(M), N]
//   wgrad:   A^T = grad_out [M_g, m_out], B^T = x [M_g, N], out = grad_w [B, m_out, N], K = M_g
// fp8 formats: 1-byte inputs, bf16 out scaled by a_scale[0] * b_scale[g] (x_scale / w_scale).
struct KernelArgs {
    const void       *x;      // A operand storage (x, or grad_out for dgrad / wgrad)
    const void       *w;      // B operand storage (w, or x for wgrad)
    void             *out;    // output, row stride N
    const GroupEntry *groups; // [group_num], device memory
    int               group_num;
    int               total_tiles; // output tiles over all groups
    int               n;           // N
    int               k;           // K (multiple of 8)
    int               n_tiles;     // ceil(N / kTileN)
    int               k_tiles;     // ceil(K / kTileK)
    int               n_xcd;       // XCDs the grid is spread over (1 = no remap)
    int               band;        // M-tiles per band of the in-group tile order
    int               lda, ldb;    // row strides (elements) of the A and B storage
    int               m_out;       // wgrad: output rows per group (0 otherwise)
    int               min_steps;   // wgrad: fewest K steps of a tile (kCrossMinStepsHost: a
                                   // cross-tile wgrad tile of a shorter group runs zero steps)
    const float      *x_scale;     // fp8: device scale of the A operand (1 value)
    const float      *w_scale;     // fp8: device scale of each group's B operand (group_num values)
    const int        *d_total;     // device tile count (device-resident group sizes), or null:
                                   // then total_tiles holds it
    int               splits;      // split-K: K ranges per tile (1 = none; per-tile variant only)
    float            *ws;          // split-K: fp32 partial sums, splits * total_tiles * 256 KB
    // In-kernel group table (device-resident sizes, group_num <= kInKernelTableGroups): every
    // wave builds its table from lens / offs at its start, with the rules of
    // build_group_table_kernel, and workgroup 0 writes the header. Null: the table in `groups`.
    const int64_t    *d_lens;      // [group_num] rows per group (device)
    const int64_t    *d_offs;      // [group_num + 1] first rows, or null for back-to-back groups
    int64_t           lens_rows;   // rows of the inputs: groups outside [0, lens_rows) are invalid
    TableHeader      *d_header;    // written by workgroup 0: tile count and the first bad group
    int               tile_n;      // output columns per tile: kTileN, kNarrowTileN (per-tile
                                   // 16-bit forward plans of one round) or kShortWideTileN
                                   // (cross-tile 16-bit forward plans of short tiles); n_tiles
                                   // counts these
    int               tile_m;      // output rows per tile: kTileM, or at most kShortTileM
                                   // (16-bit forward and dgrad plans whose groups keep their
                                   // M-tile counts; the group table counts these)
    // Tail split (cross-tile variant, host-size 16-bit forward plans with a partial last round
    // of at most half the grid): K ranges per last-round tile, 2 (1 = none). ws then holds
    // 2 * rem partial-sum slabs of 256 KB (range k of last-round tile j at slab k * rem + j), which
    // tail_reduce_kernel adds and stores after the GEMM.
    int               tail_splits;
    // Tile descriptors (null: the kernel locates its tiles itself): desc_per_wg (<= 64) entries
    // of 4 ints per workgroup, entry i of workgroup w for its tile t = w + i * grid: first row
    // of the tile in A and out, group, (N-tile << 9) | valid rows, 0. Host-size forward and
    // dgrad plans without split-K or tail split (TileDesc, built by the plan).
    const int        *desc;
    int               desc_per_wg;
    int               tails;       // 0: no partial K step and no column tail of an MN-major
                                   // operand anywhere in the plan (instances without the masks)
};

// One tile descriptor (see KernelArgs::desc).
struct TileDesc {
    int32_t row0;  // first row of the tile in A (x or grad_out) and out; wgrad: the group's first token
    int32_t g;     // group
    int32_t tn_mv; // (N-tile << 9) | valid rows (at most 256); wgrad: (N-tile << 16) | M-tile
    int32_t m;     // wgrad: the group's tokens (0 otherwise)
};
constexpr int kMaxDescPerWg = 64; // one per lane of a wave

// Tile shapes of the forward kernel: 256 x 256; narrow 256 x 224 (per-tile, one-round plans);
// short tile_m x 256 with tile_m <= kShortTileM (6 row blocks per wave); short-wide tile_m x 288
// (6 row blocks and 9 column blocks per wave; cross-tile 16-bit forward plans).
enum TileShape { kShapeWide = 0, kShapeNarrow = 1, kShapeShort = 2, kShapeShortWide = 3 };

// Fewest K steps of a tile (or tail-split K range) in the cross-tile pipeline: its first step
// plus the three whose DMAs prefetch the next tile.
constexpr int kCrossMinStepsHost = 4;

// Whether a launch takes the cross-tile pipeline variant (several tiles per workgroup, enough
// K steps) rather than a prologue and an LDS-staged epilogue per tile.
bool uses_cross_tile(const KernelArgs &args, int grid, int mode = 0);

// Launch of one kernel instance (cross-tile or per-tile variant), defined and explicitly
// instantiated in the instance units (gg_inst.hip, one (F16, MODE) pair per unit).
template <bool F16, int MODE>
void launch_mode(const KernelArgs &args, bool cross, dim3 g, dim3 b, hipStream_t stream);
// Short-tile instances (16-bit forward and dgrad; instance units of their own).
template <bool F16, int MODE>
void launch_short(const KernelArgs &args, bool cross, dim3 g, dim3 b, hipStream_t stream);
// Short-wide instances (cross-tile 16-bit forward; instance units of their own).
template <bool F16> void launch_short_wide(const KernelArgs &args, dim3 g, dim3 b, hipStream_t stream);
// Modes with short-tile instances. (fp8 forward ran 6 % slower with them on config 5a's shapes.)
constexpr bool has_short_tiles(int mode) {
    return mode == make_mode(kFwd, kIn16) || mode == make_mode(kDgrad, kIn16);
}

// Enqueue the persistent grouped GEMM: `grid` workgroups of 256 threads on `stream`.
// fp16 selects the f16 MFMA, otherwise bf16 (16-bit formats); mode = make_mode(layout, format)
// (fp8 formats write bf16, fp16 must be false).
// Returns the launch status.
hipError_t launch_grouped_gemm(const KernelArgs &args, bool fp16, int grid, hipStream_t stream,
                               int mode = 0);

// Split-K second pass: out tile = sum over the splits of the partial sums in args.ws (in split
// order), times the fp8 scales for fp8 formats, converted to 16 bits and stored within the
// tile's valid rows and columns. Forward and dgrad layouts (out row stride N).
hipError_t launch_split_reduce(const KernelArgs &args, bool fp16, hipStream_t stream, int mode = 0);

// Tail split, second pass: every last-round tile of a tail-split plan (launched on `grid`
// workgroups) = the sum of its two K ranges' partial sums in args.ws, converted to 16 bits and
// stored within the tile's valid rows and columns.
hipError_t launch_tail_reduce(const KernelArgs &args, bool fp16, int grid, hipStream_t stream);

// Build the group table on the device from device-resident group sizes: lens[group_num]
// (int64 rows) and offs[group_num + 1] (int64 first rows) or null for back-to-back groups.
// Groups outside [0, total_m) get no rows (forward / dgrad: no tiles) and are reported in the
// header. out_rows > 0 (wgrad): every group owns ceil(out_rows / 256) * n_tiles tiles. One wave.
hipError_t launch_build_group_table(const int64_t *lens, const int64_t *offs, int group_num,
                                    int64_t total_m, int n_tiles, GroupEntry *table,
                                    TableHeader *header, hipStream_t stream, int out_rows = 0);

// offs[0] = 0, offs[g + 1] = offs[g] + lens[g]: group offsets from device lengths. One wave.
hipError_t launch_group_offsets(const int64_t *lens, int64_t *offs, int group_num, hipStream_t stream);

// out[0 .. bytes) = 0 with 16-byte stores (bytes a multiple of 16), as a kernel: a caller may
// capture it in a graph, where a hipMemsetAsync node must not be recorded.
hipError_t launch_zero_fill(void *out, size_t bytes, hipStream_t stream);

// Small-tile forward plans (16-bit, host-size groups) for problems whose 256 x 256 tiles leave
// most CUs idle: 128 x 128 tiles, one per workgroup, optionally split over K.
constexpr int kSmallTile = 128; // output rows and columns of a small tile
constexpr int kSmallK    = 64;  // K per step
// LDS ring of K steps (32 KB each), DMAs S - 1 steps ahead: 4 steps (128 KB, one workgroup per
// CU) for plans of at most one tile per CU, 2 steps (64 KB, two workgroups per CU) for up to two.
constexpr int kSmallStagesOne = 4;
constexpr int kSmallStagesTwo = 2;
struct SmallTile {
    int64_t row0; // first row of the tile in x and out
    int32_t m;    // valid rows (1 .. 128)
    int16_t g;    // group (the small-tile plans take at most 32767 groups)
    int16_t tn;   // N-tile (128 columns; N <= 2^21 gives at most 16384)
};
struct SmallArgs {
    const void      *x;     // [sum(M), K]
    const void      *w;     // [B, N, K]
    void            *out;   // [sum(M), N]
    const SmallTile *tile_list; // [tiles], device memory
    float           *ws;    // split-K: splits * tiles slabs of 128 x 128 fp32 (64 KB)
    int              tiles;
    int              n, k;
    int              k_steps;         // ceil(K / 64)
    int              splits;          // K ranges per tile (1 = none)
    int              steps_per_split; // K steps per range (the last range may have fewer)
    int              stages;          // kSmallStagesOne or kSmallStagesTwo
};
// Enqueue a small-tile plan: tiles * splits workgroups of 512 threads, then (splits > 1) the
// reduction of the partial sums, one workgroup of 256 threads per tile, on the same stream.
hipError_t launch_small_gemm(const SmallArgs &args, bool fp16, hipStream_t stream);

// Seeded N(0,1) fill (benchmark input generator).
hipError_t launch_fill_randn(void *p, size_t count, uint64_t seed, bool fp16, hipStream_t stream);
hipError_t launch_clock_probe(unsigned long long *out, unsigned long long ticks, unsigned long long wall_hz,
                              hipStream_t stream);

} // namespace gg
