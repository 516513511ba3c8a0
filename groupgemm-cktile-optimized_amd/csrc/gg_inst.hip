// One instance unit of the persistent grouped GEMM: the (input type, mode) pair GG_PART selects,
// both variants (cross-tile and per-tile), (parts 14-17) the short-tile instances or (parts 18-19)
// the short-wide forward instances. 16-bit forward units also hold the cross-tile instances with
// the tail split (TAIL).
// The Makefile compiles this file once per part, in parallel; gg_kernel.hip's dispatch calls
// launch_mode of every part.
#include "gg_kernel_impl.h"

#ifndef GG_PART
#error "GG_PART selects the instance (0-19)"
#endif

namespace gg {

// Cross-tile launch of one tile shape: the instance without tail masks (KT = false) when the
// plan has no partial K step and no column tail of an MN-major operand (args.tails == 0).
template <bool F16, int MODE, int SHAPE>
void launch_cross(const KernelArgs &args, dim3 g, dim3 b, hipStream_t stream) {
    if (args.tails == 0) {
        hipLaunchKernelGGL((grouped_gemm_kernel<F16, true, MODE, SHAPE, false, false>), g, b, 0, stream, args);
        return;
    }
    hipLaunchKernelGGL((grouped_gemm_kernel<F16, true, MODE, SHAPE>), g, b, 0, stream, args);
}

template <bool F16, int MODE>
void launch_mode(const KernelArgs &args, bool cross, dim3 g, dim3 b, hipStream_t stream) {
    if constexpr (has_short_tiles(MODE)) {
        if (args.tile_m != kTileM) {
            launch_short<F16, MODE>(args, cross, g, b, stream);
            return;
        }
    }
    if (cross) {
        if constexpr (MODE == make_mode(kFwd, kIn16)) {
            if (args.tail_splits > 1) {
                hipLaunchKernelGGL((grouped_gemm_kernel<F16, true, MODE, kShapeWide, true>), g, b, 0, stream, args);
                return;
            }
        }
        launch_cross<F16, MODE, kShapeWide>(args, g, b, stream);
        return;
    }
    if constexpr (MODE == make_mode(kFwd, kIn16)) {
        // 16-bit forward per-tile plans (one round: config 5b's narrow tiles) also have instances
        // without tail masks
        if (args.tile_n == kNarrowTileN) {
            if (args.tails == 0)
                hipLaunchKernelGGL((grouped_gemm_kernel<F16, false, MODE, kShapeNarrow, false, false>), g, b, 0, stream, args);
            else
                hipLaunchKernelGGL((grouped_gemm_kernel<F16, false, MODE, kShapeNarrow>), g, b, 0, stream, args);
            return;
        }
        if (args.tails == 0) {
            hipLaunchKernelGGL((grouped_gemm_kernel<F16, false, MODE, kShapeWide, false, false>), g, b, 0, stream, args);
            return;
        }
    }
    hipLaunchKernelGGL((grouped_gemm_kernel<F16, false, MODE>), g, b, 0, stream, args);
}

// Defined only in the short-tile parts (14-17); launch_mode's calls in parts 0-3 link to their
// explicit instantiations, so the short-tile kernels compile once.
#if GG_PART >= 14 && GG_PART <= 17
template <bool F16, int MODE>
void launch_short(const KernelArgs &args, bool cross, dim3 g, dim3 b, hipStream_t stream) {
    if (cross) {
        if constexpr (MODE == make_mode(kFwd, kIn16)) {
            if (args.tile_n == kShortWideTileN) { // cross-tile only (launch_grouped_gemm checks)
                launch_short_wide<F16>(args, g, b, stream);
                return;
            }
            if (args.tail_splits > 1) {
                hipLaunchKernelGGL((grouped_gemm_kernel<F16, true, MODE, kShapeShort, true>), g, b, 0, stream, args);
                return;
            }
        }
        launch_cross<F16, MODE, kShapeShort>(args, g, b, stream);
    } else
        hipLaunchKernelGGL((grouped_gemm_kernel<F16, false, MODE, kShapeShort>), g, b, 0, stream, args);
}
#endif

#if GG_PART >= 18
template <bool F16> void launch_short_wide(const KernelArgs &args, dim3 g, dim3 b, hipStream_t stream) {
    launch_cross<F16, make_mode(kFwd, kIn16), kShapeShortWide>(args, g, b, stream);
}
#endif

#if GG_STAMPS
// Instrumented builds: this unit's cycle stamps (its own g_stamps) to the host, and cleared.
#define GG_STAMP_CAT2(a, b) a##b
#define GG_STAMP_CAT(a, b) GG_STAMP_CAT2(a, b)
extern "C" int GG_STAMP_CAT(gg_stamps_read_p, GG_PART)(unsigned long long *dst) {
    return static_cast<int>(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps), sizeof(g_stamps)));
}
extern "C" int GG_STAMP_CAT(gg_stamps_clear_p, GG_PART)() {
    static unsigned long long zeros[kStampWgs * kStampSlots];
    return static_cast<int>(hipMemcpyToSymbol(HIP_SYMBOL(g_stamps), zeros, sizeof(zeros)));
}
#endif

// part -> (fp16 MFMA, mode); the dispatch's switch in gg_kernel.hip covers the same 14 pairs
#if GG_PART == 0
template void launch_mode<false, make_mode(kFwd, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 1
template void launch_mode<true, make_mode(kFwd, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 2
template void launch_mode<false, make_mode(kDgrad, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 3
template void launch_mode<true, make_mode(kDgrad, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 4
template void launch_mode<false, make_mode(kWgrad, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 5
template void launch_mode<true, make_mode(kWgrad, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 6
template void launch_mode<false, make_mode(kFwd, kInE4M3)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 7
template void launch_mode<false, make_mode(kFwd, kInE5M2)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 8
template void launch_mode<false, make_mode(kDgrad, kInE4M3)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 9
template void launch_mode<false, make_mode(kDgrad, kInE5M2)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 10
template void launch_mode<false, make_mode(kDgrad, kInE5M2xE4M3)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 11
template void launch_mode<false, make_mode(kWgrad, kInE4M3)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 12
template void launch_mode<false, make_mode(kWgrad, kInE5M2)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 13
template void launch_mode<false, make_mode(kWgrad, kInE5M2xE4M3)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 14
template void launch_short<false, make_mode(kFwd, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 15
template void launch_short<true, make_mode(kFwd, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 16
template void launch_short<false, make_mode(kDgrad, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 17
template void launch_short<true, make_mode(kDgrad, kIn16)>(const KernelArgs &, bool, dim3, dim3, hipStream_t);
#elif GG_PART == 18
template void launch_short_wide<false>(const KernelArgs &, dim3, dim3, hipStream_t);
#elif GG_PART == 19
template void launch_short_wide<true>(const KernelArgs &, dim3, dim3, hipStream_t);
#else
#error "GG_PART out of range"
#endif

} // namespace gg
