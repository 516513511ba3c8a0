// Host check of the kernel's tile scheduler (gg_schedule.h is compiled here with g++, the same
// code the gfx950 kernel runs). Exit status 0 = every property holds. Checked:
//   * xcd_remap is a bijection of [0, total) that keeps every round (grid slots) inside
//     itself, and gives the workgroups of one XCD one contiguous run of logical tiles;
//   * band_coords visits every (M-tile, N-tile) of a group exactly once, and 32 consecutive
//     tiles of a full band touch at most `band` M-tiles and ceil(32 / band) + 1 N-tiles;
//   * the whole kernel walk (workgroup w handles slots w, w + grid, ...; remap; locate_tile
//     with its forward-only group hint) covers every (group, M-tile, N-tile) exactly once,
//     with empty groups owning nothing, and each workgroup's logical tiles only increase;
//   * active_rows: for every tile size (1..256 valid rows and columns, both row mappings) each
//     16 x 16 block that holds a valid output belongs to exactly one wave's active row blocks,
//     and every active block holds a valid row (no MFMA skipped that a stored output needs);
//   * band_for: 8-tile bands exactly where one group's B operand passes the Infinity Cache;
//   * desc_rows_fit: tile descriptors (32-bit first rows) are refused when a wgrad plan's input
//     tokens pass 2^31 although its output rows (group_num * N) are few, and accepted when every
//     group's first token from build_group_table fits.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <tuple>
#include <vector>

#include "gg_schedule.h"

static int failures = 0;
#define CHECK(cond, ...)                                                                      \
    do {                                                                                      \
        if (!(cond)) {                                                                        \
            if (failures < 20) {                                                              \
                std::printf("FAIL %s:%d: ", __FILE__, __LINE__);                              \
                std::printf(__VA_ARGS__);                                                     \
                std::printf("\n");                                                            \
            }                                                                                 \
            ++failures;                                                                       \
        }                                                                                     \
    } while (0)

static void check_remap(int total, int grid, int n_xcd) {
    std::vector<int> seen(total, 0);
    for (int t = 0; t < total; ++t) {
        const int L = gg::xcd_remap(t, total, grid, n_xcd);
        CHECK(L >= 0 && L < total, "remap out of range t=%d total=%d grid=%d", t, total, grid);
        if (L < 0 || L >= total)
            continue;
        CHECK(L / grid == t / grid, "remap leaves its round t=%d L=%d grid=%d", t, L, grid);
        ++seen[L];
    }
    for (int L = 0; L < total; ++L)
        CHECK(seen[L] == 1, "logical tile %d hit %d times (total=%d grid=%d xcd=%d)", L, seen[L],
              total, grid, n_xcd);
    if (n_xcd > 1 && grid % n_xcd == 0) {
        // contiguity: per round and XCD, the logical tiles form one interval
        for (int base = 0; base < total; base += grid) {
            for (int x = 0; x < n_xcd; ++x) {
                int lo = total, hi = -1, cnt = 0;
                for (int i = x; i < grid && base + i < total; i += n_xcd) {
                    const int L = gg::xcd_remap(base + i, total, grid, n_xcd);
                    lo = L < lo ? L : lo;
                    hi = L > hi ? L : hi;
                    ++cnt;
                }
                CHECK(cnt == 0 || hi - lo + 1 == cnt, "XCD %d of round %d not contiguous", x,
                      base / grid);
            }
        }
    }
}

static void check_band(int m_tiles, int n_tiles, int band) {
    std::set<std::pair<int, int>> seen;
    const int total = m_tiles * n_tiles;
    for (int i = 0; i < total; ++i) {
        int tm, tn;
        gg::band_coords(i, m_tiles, n_tiles, band, &tm, &tn);
        CHECK(tm >= 0 && tm < m_tiles && tn >= 0 && tn < n_tiles, "band coords out of range");
        CHECK(seen.insert({tm, tn}).second, "tile (%d,%d) visited twice", tm, tn);
    }
    CHECK((int)seen.size() == total, "band order misses tiles");
    // locality inside full bands
    const int full_bands = m_tiles / band;
    for (int b = 0; b < full_bands; ++b)
        for (int s = b * band * n_tiles; s + 32 <= (b + 1) * band * n_tiles; s += 32) {
            std::set<int> ms, ns;
            for (int i = s; i < s + 32; ++i) {
                int tm, tn;
                gg::band_coords(i, m_tiles, n_tiles, band, &tm, &tn);
                ms.insert(tm);
                ns.insert(tn);
            }
            CHECK((int)ms.size() <= band && (int)ns.size() <= (32 + band - 1) / band + 1,
                  "32 consecutive tiles touch %zu M-tiles and %zu N-tiles", ms.size(), ns.size());
        }
}

// out_rows > 0: the weight-gradient walk, where every group (empty ones included) owns an
// out_rows x n output.
// tile_m: rows per M-tile (short tiles: fewer than 256).
static void check_walk(const std::vector<int64_t> &group_m, int64_t n, int grid, int n_xcd,
                       int64_t out_rows = 0, int tile_m = gg::kTileM, int band = gg::kBand) {
    const int64_t n_tiles = gg::cdiv(n, gg::kTileN);
    std::vector<gg::GroupEntry> table(group_m.size());
    const int64_t total = gg::build_group_table(group_m.data(), (int)group_m.size(), n_tiles,
                                                table.data(), out_rows, tile_m);
    CHECK(total >= 0, "table build failed");
    std::set<std::tuple<int, int, int>> seen;
    for (int wg = 0; wg < grid; ++wg) {
        int g = 0, prevL = -1;
        for (int t = wg; t < total; t += grid) {
            const int L = gg::xcd_remap(t, (int)total, grid, n_xcd);
            CHECK(L > prevL, "logical tiles of workgroup %d not increasing", wg);
            prevL = L;
            int tm, tn;
            gg::locate_tile(L, table.data(), (int)group_m.size(), (int)n_tiles, band, &g, &tm,
                            &tn, (int)out_rows, tile_m);
            const int64_t rows = out_rows > 0 ? out_rows : group_m[g];
            CHECK(rows > 0, "tile assigned to empty group %d", g);
            CHECK(tm * tile_m < rows && tn * gg::kTileN < n, "tile outside group");
            CHECK(seen.insert({g, tm, tn}).second, "tile (%d,%d,%d) twice", g, tm, tn);
        }
    }
    int64_t want = 0;
    for (int64_t m : group_m)
        want += gg::cdiv(out_rows > 0 ? out_rows : m, tile_m) * n_tiles;
    CHECK((int64_t)seen.size() == want && want == total, "walk covers %zu of %lld tiles",
          seen.size(), (long long)want);
}

// Blocks of the 256 x 256 tile: wave (wm, wn), row block mi -> tile rows, column blocks ni of
// the wave -> columns 128 wn + 16 ni. A block with a valid output must be active in exactly one
// wave; an active block must contain a valid row and a valid column of the wave.
static void check_active_rows(bool ilv) {
    for (int mv = 1; mv <= 256; ++mv)
        for (int nv = 8; nv <= 256; nv += 8) {
            std::vector<int> cover(16 * 16, 0);
            for (int wm = 0; wm < 2; ++wm)
                for (int wn = 0; wn < 2; ++wn) {
                    const uint32_t rows = gg::active_rows(ilv, mv, nv, wm, wn);
                    CHECK((rows & (rows + 1)) == 0 && rows <= 0xffu, "row mask not a prefix: %x", rows);
                    for (int mi = 0; mi < 8; ++mi) {
                        const int r0 = ilv ? 16 * (2 * mi + wm) : 128 * wm + 16 * mi;
                        const bool act = (rows >> mi) & 1;
                        if (act)
                            CHECK(r0 < mv && 128 * wn < nv, "active block without valid output (ilv=%d m=%d n=%d wm=%d wn=%d mi=%d)",
                                  ilv, mv, nv, wm, wn, mi);
                        for (int ni = 0; ni < 8; ++ni) {
                            const int c0 = 128 * wn + 16 * ni;
                            if (act && c0 < nv)
                                ++cover[(r0 / 16) * 16 + c0 / 16];
                        }
                    }
                }
            for (int rb = 0; rb < 16; ++rb)
                for (int cb = 0; cb < 16; ++cb) {
                    const bool valid = 16 * rb < mv && 16 * cb < nv;
                    CHECK(cover[rb * 16 + cb] == (valid ? 1 : 0), "block (%d, %d) covered %d times (ilv=%d m=%d n=%d)",
                          rb, cb, cover[rb * 16 + cb], ilv, mv, nv);
                }
        }
}

// Short tiles: the rows per tile short_tile_rows picks keep every group's M-tile count and are
// the fewest (multiple of 16) that do; the short walk covers every tile once.
static void check_short(const std::vector<int64_t> &group_m, int64_t n, int want_rows) {
    const int rows = gg::short_tile_rows(group_m.data(), (int)group_m.size());
    CHECK(rows == want_rows, "short_tile_rows = %d, want %d", rows, want_rows);
    if (rows <= 0)
        return;
    CHECK(rows % 16 == 0 && rows <= gg::kShortTileM, "short rows %d", rows);
    for (int64_t m : group_m)
        CHECK(gg::cdiv(m, rows) == gg::cdiv(m, gg::kTileM), "group of %lld rows changes its tile count", (long long)m);
    bool fewer_ok = rows <= 16;
    if (!fewer_ok)
        for (int64_t m : group_m)
            if (m > 0 && gg::cdiv(m, rows - 16) != gg::cdiv(m, gg::kTileM))
                fewer_ok = true; // 16 rows fewer would add a tile to some group
    CHECK(fewer_ok, "short rows %d are not the fewest", rows);
    check_walk(group_m, n, 256, 8, 0, rows);
    check_walk(group_m, n, 24, 8, 0, rows);
}

// Descriptor row guard on a synthetic group list (no device memory: the sizes are only summed).
static void check_desc_rows() {
    // wgrad with n = k = 8: one 8 x 8 output tile per group, 20 groups of 2^27 tokens
    const std::vector<int64_t> big(20, int64_t(1) << 27);
    std::vector<gg::GroupEntry> table(big.size());
    const int64_t tiles = gg::build_group_table(big.data(), int(big.size()), 1, table.data(), 8);
    CHECK(tiles == 20, "wgrad table of 20 groups: %lld tiles", (long long)tiles);
    CHECK(table.back().row0 > INT32_MAX, "the last group's first token passes 2^31");
    CHECK(!gg::desc_rows_fit(big.data(), int(big.size()), 20 * 8), "wgrad tokens past 2^31 must not use descriptors");
    // the same groups up to the largest count whose tokens fit: every first token fits too
    const std::vector<int64_t> fits(15, int64_t(1) << 27); // 15 * 2^27 = 2^31 - 2^27
    std::vector<gg::GroupEntry> t2(fits.size());
    gg::build_group_table(fits.data(), int(fits.size()), 1, t2.data(), 8);
    CHECK(gg::desc_rows_fit(fits.data(), int(fits.size()), 15 * 8), "15 x 2^27 tokens fit");
    for (const auto &e : t2)
        CHECK(e.row0 <= INT32_MAX, "first token %lld", (long long)e.row0);
    // one token short of / at the limit, and forward plans bounded by their output rows
    const std::vector<int64_t> edge{INT32_MAX - 1};
    CHECK(gg::desc_rows_fit(edge.data(), 1, INT32_MAX - 1), "2^31 - 2 rows fit");
    const std::vector<int64_t> at{INT32_MAX};
    CHECK(!gg::desc_rows_fit(at.data(), 1, 8), "2^31 - 1 tokens do not");
    CHECK(!gg::desc_rows_fit(edge.data(), 1, INT32_MAX), "2^31 - 1 output rows do not");
    const std::vector<int64_t> neg{5, -1};
    CHECK(!gg::desc_rows_fit(neg.data(), 2, 4), "negative sizes are refused");
    CHECK(gg::desc_rows_fit(nullptr, 0, 0), "an empty plan fits");
}

int main() {
    check_desc_rows();
    check_short(std::vector<int64_t>(32, 520), 2880, 176); // config 5a: 3 x 176 instead of 256 + 256 + 8
    check_short({300, 0, 260, 130}, 1000, 160);
    check_short({100, 7, 1}, 264, 112);
    check_short({513, 1}, 512, 176);
    check_short(std::vector<int64_t>(8, 4096), 4096, 0);   // full tiles: nothing to gain
    check_short({520, 256}, 2880, 0);                      // a group of exactly 256 rows
    check_short({0, 0}, 64, 0);

    check_active_rows(true);
    check_active_rows(false);
    for (int n_xcd : {1, 8})
        for (int grid : {1, 8, 24, 100, 224, 256})
            for (int total = 1; total <= 1100; total += (total < 300 ? 1 : 37))
                check_remap(total, grid, n_xcd);
    check_remap(2048, 256, 8);
    check_remap(7168, 256, 8);
    // small-tile plans deal their whole list as one partial round of whole XCD rows
    for (int total = 1; total <= 3000; ++total)
        check_remap(total, (total + 7) / 8 * 8, 8);
    for (int band = 1; band <= 5; ++band)
        for (int m = 1; m <= 18; ++m)
            for (int nt = 1; nt <= 30; nt += 3)
                check_band(m, nt, band);
    check_band(16, 16, 4);
    check_band(16, 28, 4);
    check_band(64, 128, gg::kBandWide);
    check_band(20, 112, gg::kBandWide);
    // band_for: 8-tile bands only where one group's B operand is larger than the Infinity Cache
    CHECK(gg::band_for(32768, 8192, 2) == gg::kBandWide, "w of 512 MB keeps 4-tile bands");
    CHECK(gg::band_for(32768, 6144, 2) == gg::kBandWide, "w of 384 MB keeps 4-tile bands");
    CHECK(gg::band_for(8192, 16384, 2) == gg::kBand, "w of exactly 256 MB takes 8-tile bands");
    CHECK(gg::band_for(28672, 4096, 2) == gg::kBand, "w of 224 MB takes 8-tile bands");
    CHECK(gg::band_for(32768, 8192, 1) == gg::kBand, "fp8 w of 256 MB takes 8-tile bands");
    CHECK(gg::band_for(32768, 0, 2) == gg::kBand, "per-group contraction takes 8-tile bands");
    CHECK(gg::band_for(int64_t(1) << 21, int64_t(1) << 21, 2) == gg::kBandWide, "largest shape");
    // the BASELINE configs and ragged / empty groups
    check_walk(std::vector<int64_t>(4, 256), 512, 8, 8);
    check_walk(std::vector<int64_t>(8, 4096), 4096, 256, 8);
    check_walk(std::vector<int64_t>(8, 4096), 7168, 256, 8);
    check_walk(std::vector<int64_t>(32, 520), 2880, 256, 8);
    check_walk(std::vector<int64_t>(1, 2048), 7168, 224, 8);
    check_walk({0, 300, 0, 0, 1, 2000, 0}, 1000, 17, 1);
    check_walk({0, 300, 0, 0, 1, 2000, 0}, 1000, 24, 8);
    check_walk({257, 0, 255, 4096, 3}, 264, 256, 8);
    // weight gradient: every group owns out_rows x n, empty groups included
    check_walk(std::vector<int64_t>(8, 4096), 7168, 256, 8, 4096);
    check_walk({0, 300, 0, 0, 1, 2000, 0}, 1000, 24, 8, 776);
    check_walk({0, 0, 0}, 64, 3, 1, 64);
    check_walk({520, 0, 520}, 2880, 256, 8, 2880);
    // 8-tile bands: single GEMMs whose w outgrows the Infinity Cache, and ragged groups
    check_walk({4096}, 32768, 256, 8, 0, gg::kTileM, gg::kBandWide);
    check_walk({16384}, 32768, 256, 8, 0, gg::kTileM, gg::kBandWide);
    check_walk({0, 300, 0, 0, 1, 2000, 0}, 1000, 24, 8, 0, gg::kTileM, gg::kBandWide);
    check_walk({257, 0, 255, 4096, 3}, 264, 256, 8, 0, gg::kTileM, gg::kBandWide);
    if (failures) {
        std::printf("%d failures\n", failures);
        return 1;
    }
    std::printf("schedule OK\n");
    return 0;
}
