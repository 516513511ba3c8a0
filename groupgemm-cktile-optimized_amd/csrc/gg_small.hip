// Small-tile forward kernel (16-bit inputs and output, out[g] = x[g] @ w[g]^T, RCR) for problems
// whose 256 x 256 tiles cannot fill the GPU: one 128 x 128 output tile, or one K range of it
// (split-K), per workgroup of 512 threads.
//
// Operands go from global memory to LDS by DMA (buffer_load ... lds, 16 bytes per lane) into a
// ring of S K steps of 64, issued S - 1 steps ahead: S = 4 (128 KB, one workgroup per CU) for
// plans of at most one tile per CU, S = 2 (64 KB, two workgroups per CU, 97 registers per lane)
// for up to two. Rows are 128 bytes in LDS, their 16-byte pieces
// stored at (piece ^ (row % 8)) so that 8 lanes reading 8 consecutive rows hit 8 different bank
// groups. Eight waves, two per SIMD: waves 0-3 multiply the first 32 K of every step and waves
// 4-7 the second, each for a 64 x 64 quarter of the tile, with v_mfma_f32_16x16x32 (bf16 or
// f16); while one wave of a SIMD waits on its LDS reads the other issues MFMAs. w rows are the
// first source and x rows the second, so a lane's 4 accumulators are 4 consecutive output
// columns of one row (one 8-byte store). The two K halves are added through LDS at the end.
//
// Bounds: the x and w resources end at the tile's last valid row (loads past it return 0); a
// row piece past K (K % 64 != 0), which would read the next row, is loaded from an offset past
// the resource instead (zeros).
// Stores are masked by valid row and column (N % 8 == 0: four columns are all valid or not).
// Split-K: each K range writes its fp32 accumulators to a 64 KB slab in lane order, and
// small_reduce_kernel adds the slabs of a tile in split order (deterministic) and stores.
#include "gg_kernel.h"

namespace gg {
namespace {

typedef __bf16   sbf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 sf16x8 __attribute__((ext_vector_type(8)));
typedef float    sf32x4 __attribute__((ext_vector_type(4)));
typedef unsigned su32x4 __attribute__((ext_vector_type(4)));
typedef unsigned su32x2 __attribute__((ext_vector_type(2)));
typedef int      si32x4 __attribute__((ext_vector_type(4)));

constexpr int kStage = kSmallTile * 128; // bytes of one operand's K step in LDS (16 KB)

template <bool F16> __device__ __forceinline__ sf32x4 mma(const su32x4 &b, const su32x4 &a, const sf32x4 &c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(sf16x8, b), __builtin_bit_cast(sf16x8, a),
                                                      c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sbf16x8, b),
                                                       __builtin_bit_cast(sbf16x8, a), c, 0, 0, 0);
}

template <bool F16> __device__ __forceinline__ su32x2 to16(const sf32x4 &v) {
    su32x2 r;
    if constexpr (F16) {
        r[0] = __builtin_bit_cast(unsigned, (_Float16 __attribute__((ext_vector_type(2)))){(_Float16)v[0], (_Float16)v[1]});
        r[1] = __builtin_bit_cast(unsigned, (_Float16 __attribute__((ext_vector_type(2)))){(_Float16)v[2], (_Float16)v[3]});
    } else {
        r[0] = __builtin_bit_cast(unsigned, (__bf16 __attribute__((ext_vector_type(2)))){(__bf16)v[0], (__bf16)v[1]});
        r[1] = __builtin_bit_cast(unsigned, (__bf16 __attribute__((ext_vector_type(2)))){(__bf16)v[2], (__bf16)v[3]});
    }
    return r;
}

// Output row and column (within the tile) of accumulator block (i, j) of wave (wm, wn), lane l:
// row wm * 64 + 16 i + l % 16, columns wn * 64 + 16 j + 4 (l / 16) .. +3.
template <bool F16>
__device__ __forceinline__ void store_block(const SmallArgs &a, const SmallTile &t, int wm, int wn, int i, int j,
                                            int lane, const sf32x4 &v) {
    const int r  = wm * 64 + 16 * i + (lane & 15);
    const int c  = wn * 64 + 16 * j + 4 * (lane >> 4);
    const int nv = a.n - t.tn * kSmallTile;
    if (r < t.m && c < nv) {
        uint16_t *o = static_cast<uint16_t *>(a.out) + (t.row0 + r) * static_cast<int64_t>(a.n) +
                      static_cast<int64_t>(t.tn) * kSmallTile + c;
        *reinterpret_cast<su32x2 *>(o) = to16<F16>(v);
    }
}

// 64 lanes x 16 bytes from the buffer (per-lane byte offset) into LDS at lds_dst + 16 * lane.
// The M0 write must precede the LDS DMA by 5 wait states (s_nop 4), which also covers a resource
// SGPR written by a VALU instruction (v_readfirstlane) just before. The compiler does not see
// the LDS write: the K loop waits on vmcnt by hand before the barrier that publishes it.
__device__ __forceinline__ void dma16(uint32_t lds_dst, int voff, const si32x4 &rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\t"
                 "s_nop 4\n\t"
                 "buffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_dst), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// This wave's DMAs have at most VM of its vector-memory loads outstanding, its LDS reads are
// done, and so are every other wave's (barrier).
template <int VM> __device__ __forceinline__ void wait_vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

__device__ __forceinline__ si32x4 raw_rsrc(const void *p, int bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    si32x4         r;
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v)));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane(bytes);
    r[3] = 0x00020000;
    return r;
}

template <bool F16, bool SPLIT, int S>
__global__ void __launch_bounds__(512, S == kSmallStagesTwo ? 4 : 2) small_gemm_kernel(const SmallArgs a) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[S][2][kStage]; // [stage][x, w]
    // wave is uniform: readfirstlane keeps it (and the DMAs' LDS addresses) in SGPRs
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wave >> 2, wq = wave & 3; // K half of every step, quarter of the tile
    const int wm = wq >> 1, wn = wq & 1;
    const int tile  = static_cast<int>(blockIdx.x) % a.tiles;
    const int split = static_cast<int>(blockIdx.x) / a.tiles;
    const SmallTile t = a.tile_list[tile];
    const int       K = a.k;
    const int       nv = min(kSmallTile, a.n - t.tn * kSmallTile);
    const int       s0 = split * a.steps_per_split;
    const int       s1 = min(a.k_steps, s0 + a.steps_per_split);

    const char *xb = static_cast<const char *>(a.x) + t.row0 * static_cast<int64_t>(K) * 2;
    const char *wb = static_cast<const char *>(a.w) +
                     (static_cast<int64_t>(t.g) * a.n + static_cast<int64_t>(t.tn) * kSmallTile) * K * 2;
    const si32x4 xr = raw_rsrc(xb, t.m * K * 2);
    const si32x4 wr = raw_rsrc(wb, nv * K * 2);

    // DMA d (0..15) of an operand fills rows 8 d .. 8 d + 7 (1 KB): lane l takes row 8 d + l / 8
    // and the K piece (l % 8) ^ (l / 8), which lands at piece position l % 8 of that row. Wave w
    // issues DMAs 2 w and 2 w + 1 of each operand. A piece past K (K % 64 != 0), which would
    // read the next row, takes an offset past both resources (at most 128 * 2^21 * 2 = 2^29
    // bytes), so the DMA writes zeros.
    const int      drow = lane >> 3, dpiece = (lane & 7) ^ drow;
    const int      dbase = (wave * 16 + drow) * K * 2 + dpiece * 16;
    const uint32_t lds0  = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&lds[0][0][0]));
    auto issue = [&](int s) {
        const uint32_t st  = lds0 + static_cast<uint32_t>(s % S) * (2 * kStage) + wave * 2048;
        const int      oob = ((K - 1 - s * kSmallK - dpiece * 8) >> 31) & 0x40000000;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int off = (dbase + j * 8 * K * 2 + s * 128) | oob;
            dma16(st + j * 1024, off, xr);
            dma16(st + kStage + j * 1024, off, wr);
        }
    };

    sf32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = sf32x4{0.f, 0.f, 0.f, 0.f};

    // Eight waves, two per SIMD: waves 0-3 take the first 32 K of every step and waves 4-7 the
    // second, each for its quarter (wm, wn) of the tile; the two halves are added at the end.
    // Fragment reads: row (wm or wn) * 64 + 16 i + lane % 16, piece 4 kh + lane / 16.
    // The ring: step s in stage s % S, its DMAs issued S - 1 steps ahead, right after the barrier
    // that ends every wave's reads of the stage they overwrite (step s - 1's).
    const int frow = lane & 15, fpiece = lane >> 4;
    const int p    = ((4 * kh + fpiece) ^ (frow & 7)) << 4;
    for (int s = s0; s < min(s1, s0 + S - 1); ++s)
        issue(s);
    for (int s = s0; s < s1; ++s) {
        if (S > 2 && s + S - 2 < s1) // the DMAs of steps s + 1 .. s + S - 2 (4 per step and wave) may run on
            wait_vm_barrier<(S > 2 ? S - 2 : 0) * 4>();
        else
            wait_vm_barrier<0>();
        if (s + S - 1 < s1)
            issue(s + S - 1);
        const unsigned char *sa = &lds[s % S][0][0];
        su32x4               fa[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            fa[i] = *reinterpret_cast<const su32x4 *>(sa + (wm * 64 + 16 * i + frow) * 128 + p);
        // one w fragment at a time: 20 fragment registers instead of 32 (two workgroups per CU
        // with a 2-step ring leave 128 registers per lane)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const su32x4 fb = *reinterpret_cast<const su32x4 *>(sa + kStage + (wn * 64 + 16 * j + frow) * 128 + p);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j] = mma<F16>(fb, fa[i], acc[i][j]);
        }
    }

    // 20 wait states between the last MFMA and the first read of its accumulators (gfx950 needs
    // up to 19 after a 16-pass MFMA; the build's hazard scan counts each MFMA issue as 4)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory");
    // The second K halves through LDS (the ring is free: every DMA has landed and been read):
    // waves 4-7 write theirs, waves 0-3 add them to their own (first half + second half).
    float *red = reinterpret_cast<float *>(&lds[0][0][0]);
    __syncthreads();
    if (kh == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<sf32x4 *>(red + ((wq * 16 + i * 4 + j) * 64 + lane) * 4) = acc[i][j];
    }
    __syncthreads();
    if (kh == 1)
        return;
    // Add the second K half and store (or write the range's slab) one row of blocks at a time,
    // so that few loaded values are in flight beside the accumulators.
    float *slab = SPLIT ? a.ws + (static_cast<int64_t>(split) * a.tiles + tile) * (kSmallTile * kSmallTile) : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int    q = ((wq * 16 + i * 4 + j) * 64 + lane) * 4;
            const sf32x4 v = acc[i][j] + *reinterpret_cast<const sf32x4 *>(red + q);
            if constexpr (SPLIT)
                *reinterpret_cast<sf32x4 *>(slab + q) = v;
            else
                store_block<F16>(a, t, wm, wn, i, j, lane, v);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Split-K second pass: one workgroup per tile; each thread adds its 16 accumulator blocks over
// the splits, in split order, and stores them where the unsplit kernel would.
template <bool F16> __global__ void __launch_bounds__(256) small_reduce_kernel(const SmallArgs a) {
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const int tile = static_cast<int>(blockIdx.x);
    const SmallTile t    = a.tile_list[tile];
    const int64_t   slab = static_cast<int64_t>(a.tiles) * (kSmallTile * kSmallTile);
    const float    *src  = a.ws + static_cast<int64_t>(tile) * (kSmallTile * kSmallTile);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int p   = ((wave * 16 + i * 4 + j) * 64 + lane) * 4;
            sf32x4    sum = *reinterpret_cast<const sf32x4 *>(src + p);
            for (int s = 1; s < a.splits; ++s)
                sum += *reinterpret_cast<const sf32x4 *>(src + s * slab + p);
            store_block<F16>(a, t, wave >> 1, wave & 1, i, j, lane, sum);
        }
}

} // namespace

template <bool F16, bool SPLIT>
void launch_ring(const SmallArgs &a, dim3 grid, dim3 block, hipStream_t stream) {
    if (a.stages == kSmallStagesTwo)
        small_gemm_kernel<F16, SPLIT, kSmallStagesTwo><<<grid, block, 0, stream>>>(a);
    else
        small_gemm_kernel<F16, SPLIT, kSmallStagesOne><<<grid, block, 0, stream>>>(a);
}

hipError_t launch_small_gemm(const SmallArgs &a, bool fp16, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(a.tiles * a.splits)), block(512), rblock(256);
    if (a.stages != kSmallStagesOne && a.stages != kSmallStagesTwo)
        return hipErrorInvalidValue;
    if (a.splits > 1) {
        if (fp16)
            launch_ring<true, true>(a, grid, block, stream);
        else
            launch_ring<false, true>(a, grid, block, stream);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return e;
        if (fp16)
            small_reduce_kernel<true><<<dim3(a.tiles), rblock, 0, stream>>>(a);
        else
            small_reduce_kernel<false><<<dim3(a.tiles), rblock, 0, stream>>>(a);
    } else if (fp16) {
        launch_ring<true, false>(a, grid, block, stream);
    } else {
        launch_ring<false, false>(a, grid, block, stream);
    }
    return hipGetLastError();
}

} // namespace gg
