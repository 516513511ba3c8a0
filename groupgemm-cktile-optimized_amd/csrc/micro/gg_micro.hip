// Microbenchmarks behind the kernel's operand layouts (gfx950, 256 workgroups x 4 waves, one per
// CU): what an LDS DMA costs the CU's vector-memory unit by the way its 64 lanes address global
// memory, and what a transposed LDS read costs by the way its lanes address LDS. Every address
// stays inside the buffers below; each kernel ends after a fixed number of iterations.
//   ./bin/gg_micro            -> one line per pattern: cycles per instruction per CU
// C-tile stores run on all 256 CUs (st256) and on 64 (st 64).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

namespace {

typedef int   i32x2 __attribute__((ext_vector_type(2)));
typedef int   i32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kGrid = 256, kIters = 2000;
constexpr int kLd = 8192, kRows = 2048; // DMA source: 2048 rows of 8 KB (16 MB)

// ---- LDS DMA: buffer_load_dwordx4 ... lds, 16 bytes per lane, 1 KB per instruction ----------
enum DmaPattern { kDmaKMajor, kDmaRowPerLane, kDmaTwoLanesPerRow, kDmaRowPer16Lanes, kDmaPatterns };
const char *kDmaNames[kDmaPatterns] = {
    "K-major: 8 rows x 128 B, 8 lanes per row (x, w of the forward op)",
    "MN-major, a stored row per lane: 8 rows x 128 B, lane%8 = row",
    "16-bit MN-major: 4 rows x 256 B, 2 lanes per 32 B of a row",
    "fp8 MN-major: 4 rows x 256 B, 16 lanes per row (4 per 64 B)",
};

// Byte offset of lane l of DMA j of wave w within one K step (at most 256 rows).
__device__ int dma_lane(int pat, int w, int j, int l) {
    switch (pat) {
    case kDmaKMajor: return (8 * (4 * j + w) + (l >> 3)) * kLd + ((l & 7) ^ (l >> 3)) * 16;
    case kDmaRowPerLane: return (8 * (4 * j + w) + (l & 7)) * kLd + ((w & 1) * 8 + (l >> 3)) * 16;
    case kDmaTwoLanesPerRow:
        return (4 * (4 * j + w) + ((l & 7) >> 1)) * kLd + ((w & 1) * 8 + (l >> 3)) * 32 + (l & 1) * 16;
    default: {
        // the kernel's fp8 MN-major lane offset (gg_kernel_impl.h, dma_off): 128 rows per K step
        const int sw = (j >> 1) & 1, rlo = (4 * w + (l >> 4)) & 7;
        return (16 * (j ^ sw) + 4 * w + (l >> 4)) * kLd + (8 * (((l & 15) >> 3) ^ sw) + ((l & 7) ^ rlo)) * 16;
    }
    }
}

__device__ i32x4 make_rsrc(const void *p, unsigned bytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(p);
    i32x4 r;
    r[0] = static_cast<int>(static_cast<unsigned>(a));
    r[1] = static_cast<int>(static_cast<unsigned>(a >> 32) & 0xffffu);
    r[2] = static_cast<int>(bytes);
    r[3] = 0x00020000;
    return r;
}

template <int PAT>
__global__ __launch_bounds__(256) void dma_kernel(const char *buf, unsigned long long *cyc) {
    __shared__ __attribute__((aligned(16))) char smem[32768];
    const int   lane = threadIdx.x & 63;
    const int   wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const i32x4 rs   = make_rsrc(buf, static_cast<unsigned>(kLd) * kRows);
    const int   soff = 0;
    const unsigned lds0 = static_cast<unsigned>(reinterpret_cast<size_t>(smem));
    int lane_off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) lane_off[j] = dma_lane(PAT, wave, j, lane);
    __syncthreads();
    const unsigned long long t0 = __builtin_readcyclecounter();
    for (int it = 0; it < kIters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // the K step's first row; every lane stays below row 256 of it (< kRows)
            const int      r0   = (it * 256 + static_cast<int>(blockIdx.x) * 16) % (kRows - 256);
            const int      voff = r0 * kLd + lane_off[j];
            const unsigned m0   = lds0 + wave * 1024 + j * 4096; // < 32 KB
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :
                         : "s"(m0), "v"(voff), "s"(rs), "s"(soff)
                         : "memory", "m0");
        }
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const unsigned long long t1 = __builtin_readcyclecounter();
    if (threadIdx.x == 0)
        cyc[blockIdx.x] = t1 - t0;
}

// ---- transposed LDS reads: ds_read_b64_tr_b8 / ds_read_b64_tr_b16 -----------------------------
enum TrPattern { kTr8Contig, kTr8RowStride, kTr16Contig, kTr16RowStride, kTr8Kernel, kTr16Kernel, kTrPatterns };
const char *kTrNames[kTrPatterns] = {
    "tr_b8, group reads 128 contiguous bytes",
    "tr_b8, group reads 8 rows of 16 B at a 128-byte row stride",
    "tr_b16, group reads 128 contiguous bytes",
    "tr_b16, group reads 4 rows of 32 B at a 128-byte row stride",
    "tr_b8, the kernel's fp8 MN-major fragment reads",
    "tr_b16, the kernel's 16-bit MN-major fragment reads",
};

// LDS byte address of lane l in read r (0-15: block r % 8, k-half / half from r / 8 and the wave).
__device__ int tr_lane(int pat, int w, int l, int r) {
    const int q = l >> 4, s = l & 15, blk = r & 7, kh = (r >> 3) & 1, half = (w >> 1) & 1, h = w & 1;
    switch (pat) {
    case kTr8Contig:
    case kTr16Contig: return w * 4096 + l * 8 + (r & 3) * 512 + (r >> 2) * 16;
    case kTr8RowStride: return w * 4096 + (s >> 1) * 128 + (s & 1) * 8 + q * 2048 + (r & 3) * 512 + (r >> 2) * 16;
    case kTr16RowStride: return w * 4096 + (s >> 2) * 128 + (s & 3) * 8 + q * 2048 + (r & 3) * 512 + (r >> 2) * 16;
    case kTr8Kernel: {
        // gg_kernel_impl.h: fragment base of an fp8 MN-major operand, slot XOR, k-half and half offsets
        const int base = q * 8192 + (s >> 1) * (256 + 16) + (s & 1) * 8 + 128 * (h ^ (q & 1));
        return (base ^ (16 * blk)) + kh * 4096 + half * 2048;
    }
    default: {
        const int base = h * 1024 + q * 4096 + s * 8 + ((blk & 1) ? -128 : 128) * (q & 1);
        return base + kh * 16384 + half * 2048 + blk * 128;
    }
    }
}

template <int PAT>
__global__ __launch_bounds__(256) void tr_kernel(int *out, unsigned long long *cyc) {
    __shared__ __attribute__((aligned(16))) char smem[32768];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 32768 / 4; i += 256)
        reinterpret_cast<int *>(smem)[i] = i * 2654435761u;
    __syncthreads();
    int a[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = tr_lane(PAT, wave, lane, r); // all < 32 KB - 8
    int acc0 = 0, acc1 = 0;
    const unsigned long long t0 = __builtin_readcyclecounter();
    for (int it = 0; it < kIters; ++it) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            i32x2 v;
            if constexpr (PAT == kTr8Contig || PAT == kTr8RowStride || PAT == kTr8Kernel)
                v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2 *)(smem + a[r]));
            else
                v = __builtin_bit_cast(i32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(smem + a[r])));
            acc0 ^= v[0];
            acc1 += v[1];
        }
        asm volatile("" ::: "memory");
    }
    const unsigned long long t1 = __builtin_readcyclecounter();
    out[blockIdx.x * 256 + tid] = acc0 + acc1;
    if (tid == 0)
        cyc[blockIdx.x] = t1 - t0;
}

// ---- C-tile stores: 128 buffer_store_dwordx4 (1 KB each) per workgroup, one 256 x 256 bf16 tile
// per workgroup of a 4096 x 4096 output, by lane pattern; all CUs at once or a quarter of them.
enum StorePattern { kStRowPerLane, kStRowPer8Lanes, kStorePatterns };
const char *kStoreNames[kStorePatterns] = {
    "C store, lane%8 = row: 8 rows x 128 B (the kernel's fused stores)",
    "C store, 8 consecutive lanes per row: 8 rows x 128 B",
};
constexpr int kCN = 4096, kStoreReps = 50;

template <int PAT>
__global__ __launch_bounds__(256) void store_kernel(unsigned short *c, unsigned long long *cyc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tile = static_cast<int>(blockIdx.x); // < 256: 16 x 16 tiles
    const int row0 = (tile / 16) * 256, col0 = (tile % 16) * 256;
    const int r = PAT == kStRowPerLane ? (lane & 7) : (lane >> 3);
    const int ch = PAT == kStRowPerLane ? (lane >> 3) : (lane & 7);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(c, 0, kCN * kCN * 2, 0x00020000);
    const unsigned v = static_cast<unsigned>(lane);
    const __attribute__((ext_vector_type(4))) unsigned d = {v, v + 1, v + 2, v + 3};
    const unsigned long long t0 = __builtin_readcyclecounter();
    for (int rep = 0; rep < kStoreReps; ++rep) {
        const int wr = (wave >> 1) * 128, wc = (wave & 1) * 128; // the wave's 128 x 128 quadrant
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            const int row = row0 + wr + (s >> 1) * 8 + r;          // < 4096
            const int col = col0 + wc + (s & 1) * 64 + ch * 8;    // + 8 <= 4096
            __builtin_amdgcn_raw_buffer_store_b128(d, rs, (row * kCN + col) * 2, 0, /*nt*/ 2);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const unsigned long long t1 = __builtin_readcyclecounter();
    if (threadIdx.x == 0)
        cyc[blockIdx.x] = t1 - t0;
}

#define CHECK(x)                                                                                   \
    do {                                                                                           \
        if ((x) != hipSuccess) {                                                                   \
            std::fprintf(stderr, "%s failed\n", #x);                                               \
            return 1;                                                                              \
        }                                                                                          \
    } while (0)

double mean_cycles(const unsigned long long *d, int grid = kGrid) {
    std::vector<unsigned long long> h(grid);
    if (hipMemcpy(h.data(), d, grid * 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    double s = 0;
    for (auto v : h) s += static_cast<double>(v);
    return s / grid;
}

template <int P> void launch_dma(const char *buf, unsigned long long *cyc) {
    hipLaunchKernelGGL((dma_kernel<P>), dim3(kGrid), dim3(256), 0, 0, buf, cyc);
}
template <int P> void launch_tr(int *out, unsigned long long *cyc) {
    hipLaunchKernelGGL((tr_kernel<P>), dim3(kGrid), dim3(256), 0, 0, out, cyc);
}

} // namespace

int main() {
    char *buf = nullptr;
    int  *out = nullptr;
    unsigned long long *cyc = nullptr;
    CHECK(hipMalloc(&buf, static_cast<size_t>(kLd) * kRows));
    CHECK(hipMemset(buf, 1, static_cast<size_t>(kLd) * kRows));
    CHECK(hipMalloc(&out, kGrid * 256 * 4));
    CHECK(hipMalloc(&cyc, kGrid * 8));
    using DmaFn = void (*)(const char *, unsigned long long *);
    const DmaFn dma[kDmaPatterns] = {launch_dma<0>, launch_dma<1>, launch_dma<2>, launch_dma<3>};
    for (int p = 0; p < kDmaPatterns; ++p) {
        for (int rep = 0; rep < 3; ++rep) { // the last of 3 launches
            dma[p](buf, cyc);
            CHECK(hipDeviceSynchronize());
        }
        std::printf("dma  %-70s %6.2f cycles per DMA per CU\n", kDmaNames[p], mean_cycles(cyc) / (4.0 * 8 * kIters));
    }
    using TrFn = void (*)(int *, unsigned long long *);
    const TrFn tr[kTrPatterns] = {launch_tr<0>, launch_tr<1>, launch_tr<2>, launch_tr<3>, launch_tr<4>, launch_tr<5>};
    for (int p = 0; p < kTrPatterns; ++p) {
        for (int rep = 0; rep < 3; ++rep) {
            tr[p](out, cyc);
            CHECK(hipDeviceSynchronize());
        }
        std::printf("lds  %-70s %6.2f cycles per read per CU\n", kTrNames[p], mean_cycles(cyc) / (4.0 * 16 * kIters));
    }
    unsigned short *cbuf = nullptr;
    CHECK(hipMalloc(&cbuf, static_cast<size_t>(kCN) * kCN * 2));
    for (int grid : {256, 64}) {
        for (int p = 0; p < kStorePatterns; ++p) {
            for (int rep = 0; rep < 3; ++rep) {
                if (p == kStRowPerLane)
                    hipLaunchKernelGGL((store_kernel<kStRowPerLane>), dim3(grid), dim3(256), 0, 0, cbuf, cyc);
                else
                    hipLaunchKernelGGL((store_kernel<kStRowPer8Lanes>), dim3(grid), dim3(256), 0, 0, cbuf, cyc);
                CHECK(hipDeviceSynchronize());
            }
            const double c = mean_cycles(cyc, grid) / (kStoreReps * 128.0);
            std::printf("st%3d %-70s %6.2f cycles per store per CU (%.1f B/clk per CU)\n", grid, kStoreNames[p], c,
                        1024.0 / c);
        }
    }
    return 0;
}
