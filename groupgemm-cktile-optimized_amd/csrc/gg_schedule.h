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

// Ceil division for non-negative values.
GG_HD int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Per-group entry of the device-resident group table (16 bytes). Built by the host plan
// from group_m (the reference builds the same facts per group in
// ck_grouped_gemm.cpp:166-188: row offset, M, tile range).
struct GroupEntry {
    int64_t row0;  // first row of the group in x and out
    int32_t m;     // rows (tokens) in the group; 0 for an empty group
    int32_t tile0; // first logical tile of the group
};

} // namespace gg
