// Helper kernels (split-K reduction, device group table, input generator) and the host-side
// dispatch of the persistent grouped GEMM. The GEMM kernel itself is in gg_kernel_impl.h; each
// (input type, mode) pair is compiled in its own unit (gg_inst.hip with GG_PART) so that the
// build runs in parallel.
#include "gg_kernel_impl.h"

namespace gg {
namespace {

// ---------------------------------------------------------------------------------------
// Split-K reduction: block b takes 256 16-byte positions (b % 64) of logical tile b / 64.
// Position p of a slab is wave p / 4096, accumulator block (mi, ni) = ((p / 64) % 64) / 8, % 8,
// lane p % 64, which hold C row 16 (wave / 2) + 32 mi + lane % 16 (the interleaved row blocks of a
// K-major A; split-K serves the forward and dgrad layouts only), columns
// 128 (wave % 2) + 16 ni + 4 (lane / 16) .. +3 of the tile.
// ---------------------------------------------------------------------------------------
template <bool F16, bool F8>
__global__ void __launch_bounds__(256) split_reduce_kernel(const KernelArgs args) {
    const int tile = blockIdx.x >> 6;
    int       g    = 0, tm, tn;
    locate_tile(tile, args.groups, args.group_num, args.n_tiles, args.band, &g, &tm, &tn);
    const GroupEntry ge   = args.groups[g];
    const int        p    = (blockIdx.x & 63) * 256 + static_cast<int>(threadIdx.x);
    const int        wv   = p >> 12, blk = (p >> 6) & 63, l = p & 63;
    const int        row  = (wv >> 1) * 16 + (blk >> 3) * 32 + (l & 15);
    const int        col  = (wv & 1) * 128 + (blk & 7) * 16 + (l >> 4) * 4;
    const int        N    = args.n;
    const int64_t    slab = static_cast<int64_t>(args.total_tiles) * 65536; // floats per split
    const float     *src  = args.ws + static_cast<int64_t>(tile) * 65536 + p * 4;
    // up to 8 loads in flight, then added in split order
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < args.splits; i0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (i0 + j < args.splits)
                v[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src + (i0 + j) * slab));
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (i0 + j < args.splits)
                sum = (i0 + j == 0) ? v[j] : sum + v[j];
    }
    if constexpr (F8)
        sum *= args.x_scale[0] * args.w_scale[g];
    if (row < min(kTileM, ge.m - tm * kTileM) && col < N - tn * kTileN) {
        uint16_t *o = static_cast<uint16_t *>(args.out) +
                      (ge.row0 + static_cast<int64_t>(tm) * kTileM + row) * N + static_cast<int64_t>(tn) * kTileN + col;
        *reinterpret_cast<u32x2 *>(o) = pack4<F16>(sum);
    }
}

// ---------------------------------------------------------------------------------------
// Tail split, second pass: block b takes 256 16-byte positions (b % 64) of last-round tile
// b / 64 (the tile of physical slot full + b / 64, as the GEMM's xcd_remap placed it), in the
// slab layout of split_reduce_kernel, or (CT: whole 256-row tiles with row-major accumulators,
// ct_instance) in row-major order: position p is row p / 64, columns 4 (p % 64) .. +3. The two K
// ranges are added (fp32, commutative) and stored. Short tiles store row blocks 0-5 only:
// positions of rows past tile_m are never valid rows.
// ---------------------------------------------------------------------------------------
template <bool F16, bool CT>
__global__ void __launch_bounds__(256) tail_reduce_kernel(const KernelArgs args, int grid) {
    const int j    = blockIdx.x >> 6;
    const int full = (args.total_tiles / grid) * grid;
    const int rem  = args.total_tiles - full;
    const int L    = xcd_remap(full + j, args.total_tiles, grid, args.n_xcd);
    int       g    = 0, tm, tn;
    locate_tile(L, args.groups, args.group_num, args.n_tiles, args.band, &g, &tm, &tn, 0, args.tile_m);
    const GroupEntry ge  = args.groups[g];
    const int        p   = (blockIdx.x & 63) * 256 + static_cast<int>(threadIdx.x);
    const int        wv  = p >> 12, blk = (p >> 6) & 63, l = p & 63;
    const int        row = CT ? p >> 6 : (wv >> 1) * 16 + (blk >> 3) * 32 + (l & 15);
    const int        col = CT ? (p & 63) * 4 : (wv & 1) * 128 + (blk & 7) * 16 + (l >> 4) * 4;
    const int        N   = args.n;
    const float     *src = args.ws + static_cast<int64_t>(j) * 65536 + p * 4;
    const f32x4      v0  = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src));
    const f32x4      v1  = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src + static_cast<int64_t>(rem) * 65536));
    if (row < min(args.tile_m, ge.m - tm * args.tile_m) && col < N - tn * kTileN) {
        uint16_t *o = static_cast<uint16_t *>(args.out) +
                      (ge.row0 + static_cast<int64_t>(tm) * args.tile_m + row) * N + static_cast<int64_t>(tn) * kTileN + col;
        *reinterpret_cast<u32x2 *>(o) = pack4<F16>(v0 + v1);
    }
}

// ---------------------------------------------------------------------------------------
// Group table from device-resident group sizes (one wave, groups in chunks of 64).
// The same facts as the host's build_group_table: first row, rows and first tile per group.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64)
build_group_table_kernel(const int64_t *lens, const int64_t *offs, int group_num, int64_t total_m,
                         int n_tiles, GroupEntry *table, TableHeader *header, int out_rows) {
    const int lane      = threadIdx.x;
    int64_t   row_carry = 0, tile_carry = 0;
    int       first_bad = -1;
    for (int base = 0; base < group_num; base += 64) {
        const int g     = base + lane;
        const bool live = g < group_num;
        int64_t    m    = live ? lens[g] : 0;
        bool       ok   = m >= 0 && m <= INT32_MAX;
        if (!ok)
            m = 0;
        const int64_t rows_incl = wave_inclusive_sum(m, lane);
        const int64_t row0      = offs != nullptr ? (live ? offs[g] : 0) : row_carry + rows_incl - m;
        ok = ok && row0 >= 0 && row0 <= total_m && m <= total_m - row0;
        // wgrad (out_rows > 0): every group owns the tiles of its out_rows x N output, zero
        // for a group without rows or with sizes that do not fit
        const int64_t tiles      = out_rows > 0 ? (live ? cdiv(out_rows, kTileM) * n_tiles : 0)
                                                : (ok ? cdiv(m, kTileM) * n_tiles : 0);
        const int64_t tiles_incl = wave_inclusive_sum(tiles, lane);
        if (live) {
            GroupEntry e;
            e.row0   = ok ? row0 : 0;
            e.m      = ok ? static_cast<int32_t>(m) : 0;
            e.tile0  = static_cast<int32_t>(min<int64_t>(tile_carry + tiles_incl - tiles, INT32_MAX));
            table[g] = e;
        }
        const uint64_t bad = __ballot(live && !ok);
        if (first_bad < 0 && bad != 0)
            first_bad = base + __builtin_ctzll(bad);
        row_carry += __shfl(rows_incl, 63, 64);
        tile_carry += __shfl(tiles_incl, 63, 64);
    }
    if (lane == 0) {
        const bool over     = tile_carry > INT32_MAX;
        header->total_tiles = over ? 0 : static_cast<int>(tile_carry);
        header->first_bad   = first_bad;
        header->overflow    = over ? 1 : 0;
        header->reserved    = 0;
    }
}

__global__ void __launch_bounds__(64)
group_offsets_kernel(const int64_t *lens, int64_t *offs, int group_num) {
    const int lane  = threadIdx.x;
    int64_t   carry = 0;
    if (lane == 0)
        offs[0] = 0;
    for (int base = 0; base < group_num; base += 64) {
        const int     g    = base + lane;
        const int64_t incl = wave_inclusive_sum(g < group_num ? lens[g] : 0, lane);
        if (g < group_num)
            offs[g + 1] = carry + incl;
        carry += __shfl(incl, 63, 64);
    }
}

__global__ void __launch_bounds__(256) zero_fill_kernel(u32x4 *out, size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n16; i += stride)
        out[i] = u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------------------------------
// Benchmark input generator: splitmix64 of (seed, index) -> Box-Muller N(0, 1).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <bool F16> __global__ void fill_randn_kernel(uint16_t *p, size_t n, uint64_t seed) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const uint64_t r  = splitmix64(seed ^ (i * 0x2545F4914F6CDD1Dull));
        const float    u1 = (static_cast<float>(r >> 40) + 1.0f) * (1.0f / 16777217.0f); // (0, 1]
        const float    u2 = static_cast<float>((r >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
        const float    v  = sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
        if constexpr (F16)
            p[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
        else
            p[i] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }
}

// ---------------------------------------------------------------------------------------
// Clock probe (measurement helper): one wave that sleeps in steps of about 8k cycles until
// `ticks` of the constant-rate wall clock (s_memrealtime) have passed, and records the shader
// clock counter (s_memtime) and the wall clock at both ends. Launched beside a long run of the
// GEMM (it needs a few VGPRs and no LDS, so it shares a CU with a GEMM workgroup), it gives the
// run's effective shader clock: cycles / ticks * wall_hz. out: c0, t0, c1, t1, wall_hz.
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) clock_probe_kernel(unsigned long long *out, unsigned long long ticks,
                                                          unsigned long long wall_hz) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    const unsigned long long c0 = __builtin_readcyclecounter();
    unsigned long long       t  = t0;
    while (t - t0 < ticks) {
        __builtin_amdgcn_s_sleep(127);
        t = __builtin_amdgcn_s_memrealtime();
    }
    const unsigned long long c1 = __builtin_readcyclecounter();
    const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[0] = c0;
        out[1] = t0;
        out[2] = c1;
        out[3] = t1;
        out[4] = wall_hz;
    }
}

} // namespace

bool uses_cross_tile(const KernelArgs &args, int grid, int mode) {
    // Workgroups with a single tile gain nothing from the cross-tile pipeline.
    // (a device-built table's tile count is unknown on the host: take the cross-tile variant,
    // which also handles workgroups with a single tile)
    // wgrad: every group's K-step count (the cross-tile pipeline prefetches three steps of the
    // next tile inside the current one)
    const int steps = mode_layout(mode) == kWgrad ? args.min_steps : args.k_tiles;
    return kCrossAllowed && args.splits <= 1 && steps >= kCrossMinSteps &&
           (args.d_total != nullptr || args.d_lens != nullptr || args.total_tiles > grid);
}


bool mode_supported(int mode, bool fp16) {
    switch (mode) {
    case make_mode(kFwd, kIn16):
    case make_mode(kDgrad, kIn16):
    case make_mode(kWgrad, kIn16):
        return true;
    case make_mode(kFwd, kInE4M3):
    case make_mode(kFwd, kInE5M2):
    case make_mode(kDgrad, kInE4M3):
    case make_mode(kDgrad, kInE5M2):
    case make_mode(kDgrad, kInE5M2xE4M3):
    case make_mode(kWgrad, kInE4M3):
    case make_mode(kWgrad, kInE5M2):
    case make_mode(kWgrad, kInE5M2xE4M3):
        return !fp16;
    default:
        return false;
    }
}

hipError_t launch_grouped_gemm(const KernelArgs &args, bool fp16, int grid, hipStream_t stream, int mode) {
    if (!mode_supported(mode, fp16))
        return hipErrorInvalidValue;
    // short tiles: forward and 16-bit dgrad plans with a host-built group table, never split;
    // short-wide tiles (288 columns): short cross-tile 16-bit forward plans without a tail split
    const bool wide_n = args.tile_n == kShortWideTileN;
    if (args.tile_m != kTileM &&
        (args.tile_m <= 0 || args.tile_m > kShortTileM || args.tile_m % 16 != 0 || !has_short_tiles(mode) ||
         args.d_lens != nullptr || args.d_total != nullptr || args.splits > 1 ||
         (args.tile_n != kTileN && !wide_n)))
        return hipErrorInvalidValue;
    const bool cross = uses_cross_tile(args, grid, mode);
    if (wide_n && (args.tile_m == kTileM || mode != make_mode(kFwd, kIn16) || !cross || args.tail_splits > 1))
        return hipErrorInvalidValue;
    const dim3 g(grid), b(kThreads);
#define GG_CASE(L, F)                                                                          \
    case make_mode(L, F):                                                                      \
        launch_mode<false, make_mode(L, F)>(args, cross, g, b, stream);                        \
        break;
    if (fp16) {
        switch (mode) {
        case make_mode(kFwd, kIn16): launch_mode<true, make_mode(kFwd, kIn16)>(args, cross, g, b, stream); break;
        case make_mode(kDgrad, kIn16): launch_mode<true, make_mode(kDgrad, kIn16)>(args, cross, g, b, stream); break;
        case make_mode(kWgrad, kIn16): launch_mode<true, make_mode(kWgrad, kIn16)>(args, cross, g, b, stream); break;
        }
    } else {
        switch (mode) {
            GG_CASE(kFwd, kIn16)
            GG_CASE(kDgrad, kIn16)
            GG_CASE(kWgrad, kIn16)
            GG_CASE(kFwd, kInE4M3)
            GG_CASE(kFwd, kInE5M2)
            GG_CASE(kDgrad, kInE4M3)
            GG_CASE(kDgrad, kInE5M2)
            GG_CASE(kDgrad, kInE5M2xE4M3)
            GG_CASE(kWgrad, kInE4M3)
            GG_CASE(kWgrad, kInE5M2)
            GG_CASE(kWgrad, kInE5M2xE4M3)
        }
    }
#undef GG_CASE
    return hipGetLastError();
}

hipError_t launch_tail_reduce(const KernelArgs &args, bool fp16, int grid, hipStream_t stream) {
    const int rem = args.total_tiles - (args.total_tiles / grid) * grid;
    if (rem <= 0)
        return hipSuccess;
    // the GEMM instance of whole 256-row tiles keeps row-major accumulators (ct_instance)
    const bool ct = args.tile_m == kTileM && ct_instance(make_mode(kFwd, kIn16), kShapeWide, true);
    if (fp16 && ct)
        hipLaunchKernelGGL((tail_reduce_kernel<true, true>), dim3(rem * 64), dim3(256), 0, stream, args, grid);
    else if (fp16)
        hipLaunchKernelGGL((tail_reduce_kernel<true, false>), dim3(rem * 64), dim3(256), 0, stream, args, grid);
    else if (ct)
        hipLaunchKernelGGL((tail_reduce_kernel<false, true>), dim3(rem * 64), dim3(256), 0, stream, args, grid);
    else
        hipLaunchKernelGGL((tail_reduce_kernel<false, false>), dim3(rem * 64), dim3(256), 0, stream, args, grid);
    return hipGetLastError();
}

hipError_t launch_split_reduce(const KernelArgs &args, bool fp16, hipStream_t stream, int mode) {
    const dim3 g(args.total_tiles * 64), b(256);
    if (mode_f8(mode))
        hipLaunchKernelGGL((split_reduce_kernel<false, true>), g, b, 0, stream, args);
    else if (fp16)
        hipLaunchKernelGGL((split_reduce_kernel<true, false>), g, b, 0, stream, args);
    else
        hipLaunchKernelGGL((split_reduce_kernel<false, false>), g, b, 0, stream, args);
    return hipGetLastError();
}

hipError_t launch_build_group_table(const int64_t *lens, const int64_t *offs, int group_num,
                                    int64_t total_m, int n_tiles, GroupEntry *table,
                                    TableHeader *header, hipStream_t stream, int out_rows) {
    hipLaunchKernelGGL(build_group_table_kernel, dim3(1), dim3(64), 0, stream, lens, offs,
                       group_num, total_m, n_tiles, table, header, out_rows);
    return hipGetLastError();
}

hipError_t launch_group_offsets(const int64_t *lens, int64_t *offs, int group_num, hipStream_t stream) {
    hipLaunchKernelGGL(group_offsets_kernel, dim3(1), dim3(64), 0, stream, lens, offs, group_num);
    return hipGetLastError();
}

hipError_t launch_zero_fill(void *out, size_t bytes, hipStream_t stream) {
    if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(out) & 15u) != 0)
        return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    if (n16 == 0)
        return hipSuccess;
    const size_t blocks = std::min<size_t>((n16 + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_fill_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<u32x4 *>(out), n16);
    return hipGetLastError();
}

hipError_t launch_clock_probe(unsigned long long *out, unsigned long long ticks, unsigned long long wall_hz,
                              hipStream_t stream) {
    hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, stream, out, ticks, wall_hz);
    return hipGetLastError();
}

hipError_t launch_fill_randn(void *p, size_t count, uint64_t seed, bool fp16, hipStream_t stream) {
    if (count == 0)
        return hipSuccess;
    if (fp16)
        hipLaunchKernelGGL(fill_randn_kernel<true>, dim3(4096), dim3(256), 0, stream,
                           static_cast<uint16_t *>(p), count, seed);
    else
        hipLaunchKernelGGL(fill_randn_kernel<false>, dim3(4096), dim3(256), 0, stream,
                           static_cast<uint16_t *>(p), count, seed);
    return hipGetLastError();
}

} // namespace gg
