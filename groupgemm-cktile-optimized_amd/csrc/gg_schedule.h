// Tile scheduler of the persistent grouped GEMM: which output tile a workgroup works on.
//
// Shared by the gfx950 kernel (device) and by the host (plan building, CPU unit tests), so
// the order the kernel walks is exactly the order the tests enumerate.
//
// Replaces the tile walk of the reference's persistent kernel (CK's GroupedGemmKernel loop,
// ck_grouped_gemm.cpp:97 with GemmSpatiallyLocalTilePartitioner<8,4>, config at
// ck_grouped_gemm_config.hpp:76-79). The order here is this project's own:
//
//   1. Tiles of all groups form one list; group g owns logical tiles
//      [tile0[g], tile0[g] + ceil(M_g/kTileM) * ceil(N/kTileN)).
//   2. Inside a group, tiles go in bands of `band` M-tiles; a band is walked N-tile by
//      N-tile, each N-tile top to bottom. 32 consecutive logical tiles therefore touch only
//      `band` A panels and 32/band B panels (4 + 8 = 12 for band 4).
//   3. Workgroup i of a grid of G runs on XCD i % n_xcd (the hardware dispatches
//      workgroups round-robin over the XCDs, each with its own L2). Physical tile slot t
//      (round r = t / G, workgroup i = t % G) is remapped so the workgroups of one XCD take
//      one contiguous run of logical tiles per round: their A/B panels are shared in that
//      XCD's L2 instead of being fetched by every XCD.
#pragma once

#include <stdint.h>
#include <limits.h>

#if defined(__HIPCC__)
#define GG_HD __host__ __device__ inline
#else
#define GG_HD inline
#endif

namespace gg {

constexpr int kTileM = 256; // output rows per tile (tokens)
constexpr int kTileN = 256; // output columns per tile (w rows)
constexpr int kTileK = 64;  // K per main-loop step: one 128-byte cache line per operand row
constexpr int kBand  = 4;   // M-tiles per band of the in-group order
constexpr int kBandWide = 8; // M-tiles per band when a group's B operand outgrows the Infinity Cache
constexpr int64_t kInfinityCacheBytes = int64_t(256) << 20; // MI355X: 256 MB, shared by the 8 XCDs
constexpr int kNarrowTileN = 224; // output columns of a narrow tile (one-round forward problems)
constexpr int kShortTileM  = 192; // most output rows of a short tile (6 row blocks per wave)
constexpr int kShortWideTileN = 288; // output columns of a short-wide tile (9 column blocks per wave)

// Logical tile index of physical slot `t` (t = round * grid + workgroup).
// Bijective on [0, total): every full round maps onto itself, and the last, partial round
// (total % grid slots, taken by workgroups 0 .. rem-1) maps onto [round * grid, total).
GG_HD int xcd_remap(int t, int total, int grid, int n_xcd) {
    if (n_xcd <= 1 || grid % n_xcd != 0)
        return t;
    const int round = t / grid;
    const int i     = t - round * grid; // workgroup id
    const int xcd   = i % n_xcd;
    const int local = i / n_xcd; // rank of the workgroup inside its XCD
    const int base  = round * grid;
    const int n     = total - base < grid ? total - base : grid; // slots in this round
    // Slots of this round that land on XCDs 0 .. xcd-1: XCD y gets ceil((n - y) / n_xcd).
    const int q = n / n_xcd, rem = n % n_xcd;
    const int before = xcd * q + (xcd < rem ? xcd : rem);
    return base + before + local;
}

// (M-tile, N-tile) of the tile at position `local` inside a group with m_tiles x n_tiles
// tiles, in the banded order described above.
GG_HD void band_coords(int local, int m_tiles, int n_tiles, int band, int *tm, int *tn) {
    const int per_band = band * n_tiles;
    const int b        = local / per_band;
    const int p        = local - b * per_band;
    const int left     = m_tiles - b * band;
    const int h        = left < band ? left : band; // height of this (possibly last) band
    *tn                = p / h;
    *tm                = b * band + (p - (p / h) * h);
}

// M-tiles per band for a plan whose every group multiplies by a B operand (the w rows of the
// output columns) of n x k elements of elt bytes; k = 0 where the contraction varies by group.
// With 4-tile bands one round of 256 tiles covers 4 M-tiles by 64 N-tiles: when a group's B is
// larger than the Infinity Cache, each round reads its 64 w panels from HBM and the next band
// reads them again. 8-tile bands (8 x 4 tiles per XCD: the same 12 panels per XCD and round)
// read 32 w panels per round and half the w bytes per launch.
GG_HD int band_for(int64_t n, int64_t k, int elt) {
    return n * k * elt > kInfinityCacheBytes ? kBandWide : kBand;
}

// Partial tiles: the row blocks (bit mi) of wave (wm, wn) of the 2 x 2 wave grid that hold a
// valid output in a tile of m_valid rows and n_valid columns; none when the wave's wcols columns
// (wcols wn ..: 128, or 144 in a short-wide tile) are all past n_valid. Row block mi of the wave
// is tile rows 16 (2 mi + wm) .. +16 when interleaved (ilv, a K-major A), 128 wm + 16 mi ..
// otherwise. The kernel skips the MFMAs of the other row blocks (thin K steps).
GG_HD uint32_t active_rows(bool ilv, int m_valid, int n_valid, int wm, int wn, int wcols = 128) {
    const int nb_m = (m_valid + 15) >> 4; // 16-row blocks with a valid row
    int       ra   = ilv ? (nb_m - wm + 1) >> 1 : nb_m - 8 * wm;
    ra             = ra < 0 ? 0 : (ra > 8 ? 8 : ra);
    return n_valid > wcols * wn ? (1u << ra) - 1 : 0u;
}

// Ceil division for non-negative values.
GG_HD int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Short tiles: the fewest rows per M-tile, a multiple of 16, that leave every group with the
// M-tile count of 256-row tiles; 0 when that needs more than kShortTileM rows (or no group has
// rows). A group of 520 rows takes three tiles of 176 rows instead of 256 + 256 + 8.
inline int short_tile_rows(const int64_t *group_m, int group_num) {
    int64_t rows = 0;
    for (int g = 0; g < group_num; ++g) {
        if (group_m[g] <= 0)
            continue;
        const int64_t tiles = cdiv(group_m[g], kTileM);
        const int64_t need  = cdiv(cdiv(group_m[g], tiles), 16) * 16;
        rows                = need > rows ? need : rows;
        if (rows > kShortTileM)
            return 0;
    }
    return static_cast<int>(rows);
}

// Per-group entry of the device-resident group table (16 bytes). Built by the host plan
// from group_m (the reference builds the same facts per group in
// ck_grouped_gemm.cpp:166-188: row offset, M, tile range).
struct GroupEntry {
    int64_t row0;  // first row of the group in x and out
    int32_t m;     // rows (tokens) in the group; 0 for an empty group
    int32_t tile0; // first logical tile of the group
};

// Fill `table` (group_num entries) from the group sizes; returns the total tile count, or
// -1 if a size is negative or a count overflows 32 bits. out_rows > 0: every group's output
// has out_rows rows whatever its size (the weight gradient, one [out_rows, N] block per group,
// zero for an empty group); otherwise a group's output rows are its own rows.
inline int64_t build_group_table(const int64_t *group_m, int group_num, int64_t n_tiles,
                                 GroupEntry *table, int64_t out_rows = 0, int tile_m = kTileM) {
    int64_t row = 0, tiles = 0;
    for (int g = 0; g < group_num; ++g) {
        if (group_m[g] < 0 || group_m[g] > INT32_MAX)
            return -1;
        table[g].row0  = row;
        table[g].m     = static_cast<int32_t>(group_m[g]);
        table[g].tile0 = static_cast<int32_t>(tiles);
        tiles += cdiv(out_rows > 0 ? out_rows : group_m[g], tile_m) * n_tiles;
        row += group_m[g];
        if (tiles > INT32_MAX)
            return -1;
    }
    return tiles;
}

// Whether a plan's rows fit the 32-bit first-row field of its tile descriptors (TileDesc::row0):
// forward and dgrad descriptors hold a tile's first output row (below out_rows, the plan's
// output rows), wgrad descriptors the group's first input token (below the sum of the group
// sizes, which wgrad's out_rows = group_num * N does not bound). Sizes must be >= 0.
inline bool desc_rows_fit(const int64_t *group_m, int group_num, int64_t out_rows) {
    if (out_rows >= INT32_MAX)
        return false;
    int64_t rows = 0;
    for (int g = 0; g < group_num; ++g) {
        if (group_m[g] < 0 || group_m[g] >= INT32_MAX - rows)
            return false;
        rows += group_m[g];
    }
    return true;
}

// Group and (M-tile, N-tile) of logical tile L. *g is a hint: the group of a smaller L seen
// before (0 at the start); logical tiles only grow for one workgroup, so the scan only moves
// forward. Empty groups own no tiles and are stepped over. out_rows and tile_m as in
// build_group_table. GP is a pointer to const GroupEntry in any address space (the kernel
// passes the constant address space, so the table is read with scalar loads).
template <typename GP>
GG_HD void locate_tile(int L, GP groups, int group_num, int n_tiles, int band,
                       int *g, int *tm, int *tn, int out_rows = 0, int tile_m = kTileM) {
    int gi = *g;
    while (gi + 1 < group_num && groups[gi + 1].tile0 <= L)
        ++gi;
    *g                = gi;
    const int m_tiles = ((out_rows > 0 ? out_rows : groups[gi].m) + tile_m - 1) / tile_m;
    band_coords(L - groups[gi].tile0, m_tiles, n_tiles, band, tm, tn);
}

} // namespace gg
