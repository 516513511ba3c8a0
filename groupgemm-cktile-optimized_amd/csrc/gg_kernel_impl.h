// Device code of the persistent grouped GEMM kernel. Included by the instance units
// (gg_inst.hip, one (input type, mode) pair each) and by gg_kernel.hip (helper kernels and the
// host-side dispatch).
#pragma once

// Persistent grouped GEMM for MI355X (gfx950, CDNA4): out[g] = x[g] @ w[g]^T, bf16/fp16 in,
// fp32 accumulate, bf16/fp16 out (RNE).
//
// Replaces the reference's hot path: CK's persistent GroupedGemmKernel tile loop, the
// hand-scheduled HandPipelineAsmS main loop and FastEpilogue
// (ck_kernel/ck_grouped_gemm.cpp:97, hand_pipeline_asm_s.hpp:155-357, fast_epilogue.hpp:29-118).
// Written directly against gfx950: no CK headers, no portability layers.
//
// Work decomposition
//   * Output tile 256 x 256, K step 64. One workgroup = 4 waves, one per SIMD; wave (wm, wn)
//     owns 8 x 8 MFMA blocks of 16 x 16: columns wn*128.., and the row blocks 2*mi + wm
//     (interleaved, so the valid rows of a partial tile split evenly between wm = 0 and 1;
//     contiguous rows wm*128.. for wgrad's transposed A).
//   * A wave whose blocks in a partial tile hold at most 4 row blocks with a valid output
//     skips the MFMAs of the others (thin K steps).
//   * v_mfma_f32_16x16x32_{bf16,f16}. The w fragment is the first source and the x fragment
//     the second, so each 16 x 16 accumulator holds C^T: lane l has row l%16 of the block and
//     the four consecutive columns 4*(l/16)..+3, i.e. 8 contiguous output bytes.
//   * All 256 accumulators per lane live in AGPRs (inline-asm MFMAs with "a" operands);
//     fragments, offsets and addresses use the 256 arch VGPRs.
//   * grid = min(#CUs, #tiles) persistent workgroups walking the tile list of all groups
//     (gg_schedule.h: banded in-group order + XCD remap).
//   * Two variants: cross-tile (a workgroup's tiles run as one continuous K pipeline and a
//     finished tile is stored from registers during the next tile's first step) and per-tile
//     (prologue and LDS-staged epilogue around every tile, for one tile per workgroup).
//   * Narrow tiles (kShapeNarrow, per-tile 16-bit forward only): 256 x 224, each wave 7 column
//     blocks; the host picks them for one-round plans that leave CUs idle.
//   * Short tiles (kShapeShort; 16-bit forward and dgrad): at most 192 x 256 (tile_m rows), each wave 6
//     row blocks; the host picks them when every group keeps its M-tile count (520 rows: three
//     tiles of 176 instead of 256 + 256 + 8).
//   * Short-wide tiles (kShapeShortWide; cross-tile 16-bit forward): at most 192 x 288, each wave
//     6 row blocks and 9 column blocks, on a slot plan of their own (PlanSW); the host picks them
//     when they make fewer rounds (config 5a: 960 tiles instead of 1152).
//
// LDS (160 KB, all of it): A (x rows) 2 stages + B (w rows) 3 stages of 256 rows x 128 B
// (short-wide tiles: A stages of 192 rows, B stages of 288 rows, 156 KB).
// Row r keeps its 16-byte chunk c at chunk position c ^ (r % 8): the eight lanes that a
// ds_read_b128 serves together (8 consecutive rows, same chunk) hit eight different 16-byte
// slots of a 128-byte window, which is conflict-free on gfx950.
// Global -> LDS copies use buffer_load_dwordx4 ... lds (no VGPR staging): one instruction
// moves 64 lanes x 16 B = 8 rows; lane l fetches logical chunk (l%8) ^ (l/8) of row l/8 so
// that the fixed lane -> LDS mapping (M0 + 16 l) realises the swizzle.
//
// K-step schedule (one "iteration" kt, 8 rows of 16 MFMAs per wave, see the plan_* table):
//   * x fragments are read one row ahead (2-row register ring); w fragments of step kt+1
//     are pre-read during step kt into the second half of a double-buffered register set.
//   * DMA: A(kt+1) in rows 0-2 (its first two loads were issued at the end of step kt-1),
//     B(kt+3) in rows 3-6, the first two loads of A(kt+2) at the end of row 7.
//   * One barrier per step, in row 7: after it A(kt+1) is complete in LDS, every wave is done
//     with A(kt) and with B(kt+1)'s LDS copy, so their stages can be refilled.
//   * Buffer resources are bounded by the tile's valid rows: rows past M or N read zeros and
//     are never stored. Prefetches past the last K step use a zero-length resource (no
//     traffic, the DMA writes zeros) so the DMA count, and every vmcnt, stays static.
//     K % 64 != 0: the last K step's out-of-range 16-byte chunks get an out-of-range offset.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <type_traits>

#include "gg_kernel.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace gg {
namespace {

// Pointer to const T in the constant address space (scalar loads; the data is invariant for
// the kernel's lifetime).
template <typename T> using const_space = const __attribute__((address_space(4))) T *;
template <typename T> __device__ __forceinline__ const_space<T> to_const_space(const T *p) {
    return (const_space<T>)(p);
}

typedef int      i32x2 __attribute__((ext_vector_type(2)));
typedef int      i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16   bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads  = 256;
constexpr int kWaves    = kThreads / 64;
constexpr int kRowBytes = kTileK * 2;           // 128: one K step of one operand row
constexpr int kOpBytes  = kTileM * kRowBytes;   // 32 KB: one K step of one operand tile
static_assert(kTileM == kTileN, "x and w tiles share one load layout");
constexpr int kAStages  = 2;
constexpr int kBStages  = 3;
constexpr int kLdsBytes = (kAStages + kBStages) * kOpBytes; // 163840 = all of gfx950's LDS
constexpr int kLoads    = kOpBytes / 1024 / kWaves;         // 1 KB DMAs per wave per operand step
// Slot-plan knobs (compile-time; the defaults are the tuned plan).
#ifndef GG_EARLY_A
#define GG_EARLY_A 2 // DMAs of A(kt+2) issued at the end of step kt
#endif
#ifndef GG_A_PER_ROW
#define GG_A_PER_ROW 2 // A(kt+1) DMAs per row: 2 (after MFMAs 0, 8) or 4 (0, 4, 8, 12)
#endif
#ifndef GG_B_ROW0
#define GG_B_ROW0 3 // B(kt+3) DMAs: two per row in rows GG_B_ROW0 .. +3
#endif
#ifndef GG_B_SLOT0
#define GG_B_SLOT0 0 // ... after MFMAs GG_B_SLOT0 and GG_B_SLOT0 + 8
#endif
#ifndef GG_BAR_IDX
#define GG_BAR_IDX 7 // the step's barrier follows this MFMA of row 7
#endif
#ifndef GG_M0_AHEAD
#define GG_M0_AHEAD 1 // write M0 for a DMA before the MFMA of its slot (1) or next to it (0)
#endif
#ifndef GG_ROW0_AT_BAR
#define GG_ROW0_AT_BAR 1 // next step's row-0 x fragments right after the barrier (1) or 2 slots later (0)
#endif
#ifndef GG_STAGE_BASES
#define GG_STAGE_BASES 1 // per-stage LDS base registers so every read uses the 16-bit offset field
#endif
#ifndef GG_DMA_CPOL_ID
#define GG_DMA_CPOL_ID 0 // cache-policy modifiers of the operand DMAs: see GG_DMA_CPOL
#endif
#if GG_DMA_CPOL_ID == 0
#define GG_DMA_CPOL ""
#elif GG_DMA_CPOL_ID == 1
#define GG_DMA_CPOL "nt"
#elif GG_DMA_CPOL_ID == 2
#define GG_DMA_CPOL "sc0"
#elif GG_DMA_CPOL_ID == 3
#define GG_DMA_CPOL "sc1"
#elif GG_DMA_CPOL_ID == 4
#define GG_DMA_CPOL "sc0 sc1"
#elif GG_DMA_CPOL_ID == 5
#define GG_DMA_CPOL "sc1 nt"
#endif
constexpr int kEarlyA   = GG_EARLY_A;
constexpr int kCStride  = kTileN * 2 + 16;                  // staged C row stride (528 B)
static_assert(kLoads == 8 && kEarlyA >= 0 && kEarlyA <= 4, "slot plan written for 8 DMAs per operand");
static_assert(kTileM * kCStride <= kLdsBytes, "the staged C tile must fit in LDS");

constexpr int a_stage(int s) { return s * kOpBytes; }
constexpr int b_stage(int s) { return (kAStages + s) * kOpBytes; }

// ---------------------------------------------------------------------------------------
// Operand layouts. K-major: the contraction index runs along each stored row (x and w of the
// forward op, grad_out of dgrad); a 16-row fragment k-half is one ds_read_b128. MN-major: the
// contraction index is the stored row index (w of dgrad, grad_out and x of wgrad); a fragment
// k-half is two ds_read_b64_tr_b16, each giving 4 consecutive contraction values per lane
// (fp8: a fragment is four ds_read_b64_tr_b8 of 8 values).
// A kernel mode is a layout plus an input format: mode = layout + 4 * format (gg_kernel.h).
//   layout kFwd:   out[g] = x[g] @ w[g]^T                     A = x (K-major),  B = w (K-major)
//   layout kDgrad: grad_x[g] = grad_out[g] @ w[g]             A = grad_out (K), B = w (MN)
//   layout kWgrad: grad_w[g] = grad_out[g]^T @ x[g], K = M_g  A = grad_out (MN), B = x (MN)
//   format kIn16 (bf16 / fp16), kInE4M3, kInE5M2 (both operands), kInE5M2xE4M3 (A e5m2, B
//   e4m3); fp8 formats write bf16 out = (A B^T) * a_scale * b_scale[g].
// ---------------------------------------------------------------------------------------
constexpr int  mode_layout(int m) { return m & 3; }
constexpr int  mode_fmt(int m) { return m >> 2; }
constexpr bool mode_f8(int m) { return mode_fmt(m) != kIn16; }
constexpr bool mode_a_e5(int m) { return mode_fmt(m) == kInE5M2 || mode_fmt(m) == kInE5M2xE4M3; }
constexpr bool mode_b_e5(int m) { return mode_fmt(m) == kInE5M2; }
constexpr bool mode_a_mn(int m) { return mode_layout(m) == kWgrad; }
constexpr bool mode_b_mn(int m) { return mode_layout(m) == kDgrad || mode_layout(m) == kWgrad; }
// LDS reads of one 16-row fragment over both k-halves.
constexpr int reads_per_frag(bool mn) { return mn ? 4 : 2; }

// ---------------------------------------------------------------------------------------
// Slot plan of one K step. Row mi (0..R-1) issues 16 MFMAs, idx = kh * 8 + ni; each function
// says which memory operation follows MFMA idx of row mi (-1: none). LDS reads sit after odd
// MFMAs, DMAs after even ones, so no MFMA gap holds more than one memory operation.
// NA / NB: LDS reads per fragment of A / B (2 K-major, 4 MN-major); a read op index r is the
// k-half (K-major) or k-half * 2 + half (MN-major).
// R: rows with MFMAs, 8 (256-row tiles) or 6 (short tiles). The barrier, and the next step's
// row-0 x reads behind it, sit in the last row, so MFMAs cover both whatever R is; a plan laid
// out for 8 rows would leave a short tile's last two rows of memory operations with no MFMAs
// between them, ending every step with an exposed barrier and LDS read latency.
// ---------------------------------------------------------------------------------------
static_assert(GG_BAR_IDX >= 5 && GG_BAR_IDX <= 11 && GG_BAR_IDX % 2 == 1, "barrier slot");

// First step of a cross tile: store s (0-3, see store_line) of the previous tile's row block
// mi+1 is issued after MFMA 2 + 4s of row mi (row block 0 before the step).
constexpr int plan_epi(int mi, int idx) {
    return (mi < 7 && idx % 4 == 2) ? (idx - 2) / 4 : -1;
}
template <int NA, int NB, int R = 8> struct Plan {
    static_assert(R == 8 || R == 6, "plans for 8 or 6 rows of MFMAs");
    static constexpr int rows = R, slots = 16, early = kEarlyA;
    static constexpr int nc = 8, la = kLoads, lb = kLoads; // column blocks; A / B DMAs per wave
    static constexpr int last = R - 1; // the row that holds the step's barrier
    static constexpr int epi(int mi, int idx) { return plan_epi(mi, idx); }
    // R = 8: the w fragments of row 7 are read before the barrier, at MFMAs 1 .. 2 NB - 1.
    static constexpr int bar = R < 8 || GG_BAR_IDX > 2 * NB + 1 ? GG_BAR_IDX : 2 * NB + 1;
    static constexpr int row0_first = GG_ROW0_AT_BAR ? bar : bar + 2;
    static_assert(row0_first + 2 * (NA - 1) <= 15, "row-0 reads fit in the last row");

    // x fragments of row mi+1 into the register ring: the first NA odd slots of rows 0 .. R-2.
    static constexpr int read_a_next(int mi, int idx) {
        return (mi < last && idx % 2 == 1 && idx < 2 * NA) ? idx / 2 : -1;
    }
    // R < 8: the w reads of step kt+1 (q = block * NB + read, in order) fill the odd slots after
    // the x reads of rows 0 .. R-2, spread evenly (row mi takes q in [q_first(mi), q_first(mi+1)));
    // what does not fit there takes the first odd slots of the last row, before the barrier.
    static constexpr int cap     = 8 - NA; // w-read slots of each of rows 0 .. R-2
    static constexpr int n_first = 8 * NB < (R - 1) * cap ? 8 * NB : (R - 1) * cap;
    static constexpr int q_first(int mi) { return (mi * n_first + (R - 2)) / (R - 1); }
    static constexpr int read_b_q(int mi, int idx) {
        if (idx % 2 == 0)
            return -1;
        if (mi == last) {
            const int q = n_first + idx / 2;
            return (q < 8 * NB && idx < bar) ? q : -1;
        }
        if (idx < 2 * NA)
            return -1;
        const int q = q_first(mi) + (idx - 2 * NA) / 2;
        return q < q_first(mi + 1) ? q : -1;
    }
    // w fragments of step kt+1: read op index of column block read_b_blk(mi, idx).
    // R = 8: block ni = mi, the next NB odd slots of rows 0-6; in row 7 the first NB odd slots,
    // so they are complete before the barrier.
    static constexpr int read_b_next(int mi, int idx) {
        if constexpr (R < 8) {
            return read_b_q(mi, idx) >= 0 ? read_b_q(mi, idx) % NB : -1;
        } else {
            if (idx % 2 == 0)
                return -1;
            if (mi < 7)
                return (idx >= 2 * NA && idx < 2 * (NA + NB)) ? (idx - 2 * NA) / 2 : -1;
            return idx < 2 * NB ? idx / 2 : -1;
        }
    }
    static constexpr int read_b_blk(int mi, int idx) {
        if constexpr (R < 8)
            return read_b_q(mi, idx) >= 0 ? read_b_q(mi, idx) / NB : -1;
        else
            return read_b_next(mi, idx) >= 0 ? mi : -1;
    }
    // x fragments of row 0 of step kt+1, right after the barrier.
    static constexpr int read_a_row0(int mi, int idx) {
        return (mi == last && idx % 2 == 1 && idx >= row0_first && idx < row0_first + 2 * NA)
                   ? (idx - row0_first) / 2
                   : -1;
    }
    // DMA j of A(kt+1), j = kEarlyA..7: GG_A_PER_ROW per row from row 0.
    static constexpr int load_a(int mi, int idx) {
        constexpr int per = GG_A_PER_ROW, step = 16 / per;
        if (idx % step != 0)
            return -1;
        const int j = kEarlyA + mi * per + idx / step;
        return j < kLoads ? j : -1;
    }
    // DMA j of B(kt+3). R = 8: two per row in rows GG_B_ROW0 .. +3. R < 8: four per row (after
    // MFMAs 0, 4, 8, 12) in rows 3 and 4.
    static constexpr int load_b(int mi, int idx) {
        if constexpr (R < 8)
            return (mi >= 3 && mi < 5 && idx % 4 == 0) ? (mi - 3) * 4 + idx / 4 : -1;
        else
            return (mi >= GG_B_ROW0 && mi < GG_B_ROW0 + 4 && (idx == GG_B_SLOT0 || idx == GG_B_SLOT0 + 8))
                       ? (mi - GG_B_ROW0) * 2 + (idx - GG_B_SLOT0) / 8
                       : -1;
    }
    // DMA j < kEarlyA of A(kt+2): the first even slots of the last row after the barrier (A(kt)'s
    // stage is free once every wave passed it).
    static constexpr int load_a_early(int mi, int idx) {
        const int j = (idx - (bar + 1)) / 2;
        return (mi == last && idx > bar && idx % 2 == 0 && j < kEarlyA) ? j : -1;
    }
    // The DMA that follows MFMA idx of row mi: 0 none, 1 A(kt+1), 2 B(kt+3), 3 A(kt+2).
    static constexpr int dma_kind(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? 1 : load_b(mi, idx) >= 0 ? 2 : load_a_early(mi, idx) >= 0 ? 3 : 0;
    }
    static constexpr int dma_j(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? load_a(mi, idx) : load_b(mi, idx) >= 0 ? load_b(mi, idx) : load_a_early(mi, idx);
    }
    // DMAs that may still be in flight at the barrier: those issued after the last A(kt+1)
    // DMA. Loads complete in order, so vmcnt(this) means all of A(kt+1) (and everything older)
    // landed. Stores are never counted here, wherever they sit in the step: a store may
    // complete before an older load, so counting one could let the barrier pass while an
    // A(kt+1) DMA is in flight. With loads alone counted, pending stores only make the wait
    // longer.
    static constexpr int vm_at_barrier() {
        int last_a = -1;
        for (int p = 0; p < R * 16; ++p)
            if (load_a(p / 16, p % 16) >= 0)
                last_a = p;
        int n = 0;
        for (int p = last_a + 1; p < last * 16 + bar; ++p)
            n += (load_b(p / 16, p % 16) >= 0) + (load_a_early(p / 16, p % 16) >= 0);
        return n;
    }
    template <typename F> static constexpr int count(F f) {
        int n = 0;
        for (int p = 0; p < R * 16; ++p)
            n += f(p / 16, p % 16) >= 0;
        return n;
    }
    static constexpr bool check() {
        int per_block[8] = {};
        for (int p = 0; p < R * 16; ++p) {
            const int mi = p / 16, idx = p % 16;
            const int dmas  = (load_a(mi, idx) >= 0) + (load_b(mi, idx) >= 0) + (load_a_early(mi, idx) >= 0);
            const int reads = (read_a_next(mi, idx) >= 0) + (read_b_next(mi, idx) >= 0) +
                              (read_a_row0(mi, idx) >= 0);
            if (dmas > 1 || reads > 1 || (dmas && reads))
                return false;
            // every read of step kt+1's w precedes the barrier; the row-0 x reads follow it;
            // the fused stores of a cross tile's first step (rows 0 .. R-2) meet no DMA
            if (mi == last && ((read_b_next(mi, idx) >= 0 && idx >= bar) || (read_a_row0(mi, idx) >= 0 && idx < bar)))
                return false;
            if (mi < last && epi(mi, idx) >= 0 && dmas)
                return false;
            if (read_b_next(mi, idx) >= 0) {
                const int b = read_b_blk(mi, idx);
                if (b < 0 || b > 7 || read_b_next(mi, idx) != per_block[b])
                    return false;
                ++per_block[b];
            }
        }
        for (int b = 0; b < 8; ++b)
            if (per_block[b] != NB)
                return false;
        // A(kt+1)'s DMAs all precede the barrier
        for (int p = last * 16 + bar; p < R * 16; ++p)
            if (load_a(p / 16, p % 16) >= 0)
                return false;
        return count(load_a) == kLoads - kEarlyA && count(load_b) == kLoads &&
               count(load_a_early) == kEarlyA && count(read_b_next) == 8 * NB &&
               count(read_a_next) == (R - 1) * NA && count(read_a_row0) == NA;
    }
};
static_assert(Plan<2, 2>::check() && Plan<2, 4>::check() && Plan<4, 4>::check(), "slot plans");
static_assert(Plan<2, 2, 6>::check() && Plan<2, 4, 6>::check(), "short-tile slot plans");
static_assert(Plan<2, 2, 6>::vm_at_barrier() == 8 && Plan<2, 2>::vm_at_barrier() == 8, "barrier waits");

// fp8 K step: 128 fp8 values per 128-byte row; v_mfma_f32_16x16x128_f8f6f4 takes 32 bytes of a
// row per lane, so a row mi of the step is 8 MFMAs of twice the length, and a fragment is two
// ds_read_b128 (K-major) or four ds_read_b64_tr_b8 (MN-major): NA / NB reads.
// DMAs after MFMAs 0 and 4: A(kt+1) DMAs 1-7 in rows 0-2 and row 3 (after MFMA 2), B(kt+3) in
// rows 3-6; the early A DMA 0 after MFMA 6 of row 7. The x reads of row mi+1 follow the odd
// MFMAs of row mi, the w reads of step kt+1 the MFMAs left (rows 0-6) or the first MFMAs of
// row 7, before the barrier (after MFMA 5, or 4 when row 0 of x takes four reads), and row 0 of
// the next step's x follows the barrier. A 32-cycle fp8 MFMA leaves room for a DMA or a store
// beside a read in one gap.
template <int NA, int NB> struct Plan8 {
    static_assert((NA == 2 || NA == 4) && (NB == 2 || NB == 4), "reads per fragment");
    static constexpr int rows = 8, last = 7, slots = 8, early = 1, bar = NA == 4 ? 4 : 5;
    static constexpr int nc = 8, la = kLoads, lb = kLoads;
    static constexpr int read_a_next(int mi, int idx) {
        return (mi < 7 && idx % 2 == 1 && idx < 2 * NA) ? idx / 2 : -1;
    }
    static constexpr int read_b_next(int mi, int idx) {
        if (mi == 7)
            return NB == 2 ? ((idx == 1 || idx == 3) ? idx / 2 : -1) : (idx < 4 ? idx : -1);
        if (NA == 2 && NB == 2)
            return (idx == 5 || idx == 7) ? (idx - 5) / 2 : -1;
        if (NA == 2)
            return idx == 2 ? 0 : idx == 5 ? 1 : idx == 6 ? 2 : idx == 7 ? 3 : -1;
        if (NB == 2)
            return (idx == 2 || idx == 6) ? idx / 4 : -1;
        return idx % 2 == 0 ? idx / 2 : -1;
    }
    static constexpr int read_b_blk(int mi, int idx) { return read_b_next(mi, idx) >= 0 ? mi : -1; }
    static constexpr int read_a_row0(int mi, int idx) {
        if (mi != 7)
            return -1;
        if (NA == 2)
            return (idx == 5 || idx == 7) ? (idx - 5) / 2 : -1;
        return idx >= 4 ? idx - 4 : -1;
    }
    static constexpr int load_a(int mi, int idx) {
        if (mi < 3 && (idx == 0 || idx == 4))
            return 1 + 2 * mi + idx / 4;
        return (mi == 3 && idx == 2) ? 7 : -1;
    }
    static constexpr int load_b(int mi, int idx) {
        return (mi >= 3 && mi < 7 && (idx == 0 || idx == 4)) ? 2 * (mi - 3) + idx / 4 : -1;
    }
    static constexpr int load_a_early(int mi, int idx) { return (mi == 7 && idx == 6) ? 0 : -1; }
    // Cross-tile first step: store s of the previous tile's row block mi+1 after MFMA 2, 3, 6, 7
    // of row mi.
    static constexpr int epi(int mi, int idx) {
        return mi < 7 ? (idx == 2 ? 0 : idx == 3 ? 1 : idx == 6 ? 2 : idx == 7 ? 3 : -1) : -1;
    }
    static constexpr int dma_kind(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? 1 : load_b(mi, idx) >= 0 ? 2 : load_a_early(mi, idx) >= 0 ? 3 : 0;
    }
    static constexpr int dma_j(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? load_a(mi, idx) : load_b(mi, idx) >= 0 ? load_b(mi, idx) : load_a_early(mi, idx);
    }
    static constexpr int vm_at_barrier() { // loads issued after A(kt+1)'s last DMA, as in Plan
        int last_a = -1;
        for (int p = 0; p < 8 * slots; ++p)
            if (load_a(p / slots, p % slots) >= 0)
                last_a = p;
        int n = 0;
        for (int p = last_a + 1; p < last * slots + bar; ++p)
            n += (load_b(p / slots, p % slots) >= 0) + (load_a_early(p / slots, p % slots) >= 0);
        return n;
    }
    static constexpr bool check() {
        int na = 0, nb = 0, ne = 0, ra = 0, rb = 0, r0 = 0;
        for (int p = 0; p < 8 * slots; ++p) {
            const int mi = p / slots, idx = p % slots;
            const int dmas  = (load_a(mi, idx) >= 0) + (load_b(mi, idx) >= 0) + (load_a_early(mi, idx) >= 0);
            const int reads = (read_a_next(mi, idx) >= 0) + (read_b_next(mi, idx) >= 0) + (read_a_row0(mi, idx) >= 0);
            if (dmas > 1 || reads > 1)
                return false;
            // w reads of row 7 before the barrier (reads at its slot follow it), row 0 of x after it
            if (mi == 7 && ((read_b_next(mi, idx) >= 0 && idx >= bar) || (read_a_row0(mi, idx) >= 0 && idx < bar)))
                return false;
            na += load_a(mi, idx) >= 0;
            nb += load_b(mi, idx) >= 0;
            ne += load_a_early(mi, idx) >= 0;
            ra += read_a_next(mi, idx) >= 0;
            rb += read_b_next(mi, idx) >= 0;
            r0 += read_a_row0(mi, idx) >= 0;
        }
        return na == kLoads - early && nb == kLoads && ne == early && ra == 7 * NA && rb == 8 * NB && r0 == NA;
    }
};
static_assert(Plan8<2, 2>::check() && Plan8<2, 4>::check() && Plan8<4, 4>::check(), "fp8 slot plans");
static_assert(Plan8<2, 2>::vm_at_barrier() == 7, "fp8 forward plan unchanged");
static_assert(Plan<2, 2>::bar == GG_BAR_IDX, "forward plan keeps the tuned barrier slot");

// Front-loaded slot plan of a full 16-bit K-major step (8 rows of 16 MFMAs, idx = kh * 8 + ni),
// selected by GG_PLAN=1. Each gap holds at most one memory operation, reads and DMAs in any gap:
// - the w fragments of step kt+1 in rows 0-3 (blocks 2 mi and 2 mi + 1 after MFMAs 6, 10, 12,
//   14 of rows 0-2; blocks 6 and 7 after MFMAs 3, 5, 6, 7 of row 3);
// - the x fragments of row mi+1 after MFMAs 2 and 4 of row mi;
// - A(kt+1) DMAs 2-7 after MFMAs 8 and 13 of row 0 and 0, 5, 8, 13 of row 1;
// - B(kt+3) DMAs after MFMAs 1 and 9 of rows 4-7;
// - the barrier after MFMA 10 of row 7, then row 0 of the next step's x (after MFMAs 11, 13)
//   and the early A(kt+2) DMAs 0-1 (after MFMAs 12, 14);
// - a cross tile's first step: the previous tile's row block mi+1 in four stores at the free
//   slots of row mi (epi_slot).
// A(kt+1) then has 5.5 rows to land before the barrier instead of 4.5, and the w reads are done
// before the B DMAs start.
// (Measured against it, same box, alternating, GRBM cycles: A(kt+1) after MFMAs 0, 5, 8, 13 of
// row 0 and 0, 5 of row 1: +1 to +3 %; three early A(kt+2) DMAs: +1.5 to +4 %; the barrier one
// MFMA later: -0.3 to +2 %.)
struct PlanFront {
    static constexpr int NA = 2, NB = 2;
    static constexpr int rows = 8, last = 7, slots = 16, nc = 8, early = 2, bar = 10;
    static constexpr int la = kLoads, lb = kLoads;
    static constexpr int read_a_next(int mi, int idx) { return (mi < last && (idx == 2 || idx == 4)) ? idx / 4 : -1; }
    static constexpr int b_q(int mi, int idx) { // (block << 1) | read, or -1
        if (mi < 3) {
            const int q = idx == 6 ? 0 : idx == 10 ? 1 : idx == 12 ? 2 : idx == 14 ? 3 : -1;
            return q < 0 ? -1 : ((2 * mi + q / 2) << 1) | (q & 1);
        }
        if (mi == 3) {
            const int q = idx == 3 ? 0 : idx == 5 ? 1 : idx == 6 ? 2 : idx == 7 ? 3 : -1;
            return q < 0 ? -1 : ((6 + q / 2) << 1) | (q & 1);
        }
        return -1;
    }
    static constexpr int read_b_next(int mi, int idx) { return b_q(mi, idx) >= 0 ? b_q(mi, idx) & 1 : -1; }
    static constexpr int read_b_blk(int mi, int idx) { return b_q(mi, idx) >= 0 ? b_q(mi, idx) >> 1 : -1; }
    static constexpr int read_a_row0(int mi, int idx) {
        return mi == last ? (idx == bar + 1 ? 0 : idx == bar + 3 ? 1 : -1) : -1;
    }
    static constexpr int load_a(int mi, int idx) {
        if (mi == 0)
            return idx == 8 ? 2 : idx == 13 ? 3 : -1;
        if (mi == 1)
            return idx == 0 ? 4 : idx == 5 ? 5 : idx == 8 ? 6 : idx == 13 ? 7 : -1;
        return -1;
    }
    static constexpr int load_b(int mi, int idx) {
        return (mi >= 4 && (idx == 1 || idx == 9)) ? 2 * (mi - 4) + idx / 8 : -1;
    }
    static constexpr int load_a_early(int mi, int idx) {
        return mi == last ? (idx == bar + 2 ? 0 : idx == bar + 4 ? 1 : -1) : -1;
    }
    static constexpr int epi_slot(int mi, int s) { // four free slots of each row 0-6, in order
        constexpr int lo[4] = {1, 3, 7, 11}, r3[4] = {1, 9, 11, 13}, hi[4] = {3, 7, 11, 13};
        return mi < 3 ? lo[s] : mi == 3 ? r3[s] : hi[s];
    }
    static constexpr int epi(int mi, int idx) {
        if (mi >= last)
            return -1;
        for (int s = 0; s < 4; ++s)
            if (epi_slot(mi, s) == idx)
                return s;
        return -1;
    }
    static constexpr int dma_kind(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? 1 : load_b(mi, idx) >= 0 ? 2 : load_a_early(mi, idx) >= 0 ? 3 : 0;
    }
    static constexpr int dma_j(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? load_a(mi, idx) : load_b(mi, idx) >= 0 ? load_b(mi, idx) : load_a_early(mi, idx);
    }
    static constexpr int vm_at_barrier() { // loads issued after A(kt+1)'s last DMA, as in Plan
        int last_a = -1;
        for (int p = 0; p < rows * slots; ++p)
            if (load_a(p / slots, p % slots) >= 0)
                last_a = p;
        int n = 0;
        for (int p = last_a + 1; p < last * slots + bar; ++p)
            n += (load_b(p / slots, p % slots) >= 0) + (load_a_early(p / slots, p % slots) >= 0);
        return n;
    }
    template <typename F> static constexpr int count(F f) {
        int n = 0;
        for (int p = 0; p < rows * slots; ++p)
            n += f(p / slots, p % slots) >= 0;
        return n;
    }
    static constexpr bool check() {
        int per_block[nc] = {};
        int per_row_epi[rows] = {};
        int a_seen = early;
        for (int p = 0; p < rows * slots; ++p) {
            const int mi = p / slots, idx = p % slots;
            const int ops = (load_a(mi, idx) >= 0) + (load_b(mi, idx) >= 0) + (load_a_early(mi, idx) >= 0) +
                            (read_a_next(mi, idx) >= 0) + (read_b_next(mi, idx) >= 0) +
                            (read_a_row0(mi, idx) >= 0) + (epi(mi, idx) >= 0);
            if (ops > 1)
                return false;
            // every w read of step kt+1 and every A(kt+1) DMA precede the barrier; row 0 of x
            // and the early A(kt+2) DMAs follow it
            if (p >= last * slots + bar && (read_b_next(mi, idx) >= 0 || load_a(mi, idx) >= 0))
                return false;
            if (p <= last * slots + bar && (read_a_row0(mi, idx) >= 0 || load_a_early(mi, idx) >= 0))
                return false;
            if (load_a(mi, idx) >= 0 && load_a(mi, idx) != a_seen++)
                return false;
            if (read_b_next(mi, idx) >= 0) {
                const int b = read_b_blk(mi, idx);
                if (b < 0 || b >= nc || read_b_next(mi, idx) != per_block[b])
                    return false;
                ++per_block[b];
            }
            if (epi(mi, idx) >= 0) {
                if (epi(mi, idx) != per_row_epi[mi])
                    return false;
                ++per_row_epi[mi];
            }
        }
        for (int b = 0; b < nc; ++b)
            if (per_block[b] != NB)
                return false;
        for (int r = 0; r < last; ++r)
            if (per_row_epi[r] != 4)
                return false;
        return count(load_a) == la - early && count(load_b) == lb && count(load_a_early) == early &&
               count(read_b_next) == nc * NB && count(read_a_next) == last * NA && count(read_a_row0) == NA;
    }
};
static_assert(PlanFront::check() && PlanFront::vm_at_barrier() == 8 && PlanFront::early == kEarlyA,
              "front-loaded slot plan");
#ifndef GG_PLAN
#define GG_PLAN 1 // slot plan of full 16-bit K-major steps: 0 Plan<2, 2>, 1 PlanFront
#endif

// Slot plan of a short-wide tile (at most 192 rows x 288 columns, 16-bit forward, K-major
// operands): 6 rows of 18 MFMAs per wave (9 column blocks, idx = kh * 9 + ni), A stages of 192
// rows (6 DMAs per wave) and B stages of 288 rows (9 DMAs per wave).
// - A(kt+1) DMAs 2-5 after MFMAs 0 and 10 of rows 0-1; B(kt+3) DMAs after MFMAs 0, 6 and 12 of
//   rows 2-4; the barrier after MFMA 9 of row 5, then the early A(kt+2) DMAs 0-1 (after MFMAs 10
//   and 12) and row 0 of the next step's x (after MFMAs 9 and 11).
// - The x reads of row mi+1 follow MFMAs 1 and 3 of row mi; the 18 w reads of step kt+1 the odd
//   MFMAs from 5 on of rows 0-4, spread evenly (4, 4, 3, 4, 3).
// - First step of a cross tile: store s of the previous tile's row block mi+1 after MFMA 2, 4, 8,
//   14, 16 of row mi (s = 0-3: the 8-row lines of the first 128 columns, 4: the ninth column
//   block), none next to a DMA.
struct PlanSW {
    static constexpr int NA = 2, NB = 2; // K-major reads per fragment
    static constexpr int rows = 6, last = 5, nc = 9, slots = 2 * nc, early = kEarlyA, bar = 9;
    static constexpr int la = kShortTileM * kRowBytes / 1024 / kWaves;     // 6
    static constexpr int lb = kShortWideTileN * kRowBytes / 1024 / kWaves; // 9
    static constexpr int row0_first = bar;
    static constexpr int epi(int mi, int idx) {
        if (mi >= last)
            return -1;
        return idx == 2 ? 0 : idx == 4 ? 1 : idx == 8 ? 2 : idx == 14 ? 3 : idx == 16 ? 4 : -1;
    }
    static constexpr int read_a_next(int mi, int idx) {
        return (mi < last && idx % 2 == 1 && idx < 2 * NA) ? idx / 2 : -1;
    }
    static constexpr int q_first(int mi) { return (mi * nc * NB + (rows - 2)) / (rows - 1); }
    static constexpr int read_b_q(int mi, int idx) {
        if (mi >= last || idx % 2 == 0 || idx < 2 * NA)
            return -1;
        const int q = q_first(mi) + (idx - 2 * NA) / 2;
        return q < q_first(mi + 1) ? q : -1;
    }
    static constexpr int read_b_next(int mi, int idx) { return read_b_q(mi, idx) >= 0 ? read_b_q(mi, idx) % NB : -1; }
    static constexpr int read_b_blk(int mi, int idx) { return read_b_q(mi, idx) >= 0 ? read_b_q(mi, idx) / NB : -1; }
    static constexpr int read_a_row0(int mi, int idx) {
        return (mi == last && idx % 2 == 1 && idx >= row0_first && idx < row0_first + 2 * NA)
                   ? (idx - row0_first) / 2
                   : -1;
    }
    static constexpr int load_a(int mi, int idx) {
        const int j = early + 2 * mi + idx / 10;
        return (mi < 2 && (idx == 0 || idx == 10) && j < la) ? j : -1;
    }
    static constexpr int load_b(int mi, int idx) {
        return (mi >= 2 && mi < 5 && idx % 6 == 0) ? 3 * (mi - 2) + idx / 6 : -1;
    }
    static constexpr int load_a_early(int mi, int idx) {
        const int j = (idx - (bar + 1)) / 2;
        return (mi == last && idx > bar && idx % 2 == 0 && j < early) ? j : -1;
    }
    static constexpr int dma_kind(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? 1 : load_b(mi, idx) >= 0 ? 2 : load_a_early(mi, idx) >= 0 ? 3 : 0;
    }
    static constexpr int dma_j(int mi, int idx) {
        return load_a(mi, idx) >= 0 ? load_a(mi, idx) : load_b(mi, idx) >= 0 ? load_b(mi, idx) : load_a_early(mi, idx);
    }
    static constexpr int vm_at_barrier() { // loads issued after A(kt+1)'s last DMA, as in Plan
        int last_a = -1;
        for (int p = 0; p < rows * slots; ++p)
            if (load_a(p / slots, p % slots) >= 0)
                last_a = p;
        int n = 0;
        for (int p = last_a + 1; p < last * slots + bar; ++p)
            n += (load_b(p / slots, p % slots) >= 0) + (load_a_early(p / slots, p % slots) >= 0);
        return n;
    }
    template <typename F> static constexpr int count(F f) {
        int n = 0;
        for (int p = 0; p < rows * slots; ++p)
            n += f(p / slots, p % slots) >= 0;
        return n;
    }
    static constexpr bool check() {
        int per_block[nc] = {};
        int per_row_epi[rows] = {};
        for (int p = 0; p < rows * slots; ++p) {
            const int mi = p / slots, idx = p % slots;
            const int dmas  = (load_a(mi, idx) >= 0) + (load_b(mi, idx) >= 0) + (load_a_early(mi, idx) >= 0);
            const int reads = (read_a_next(mi, idx) >= 0) + (read_b_next(mi, idx) >= 0) +
                              (read_a_row0(mi, idx) >= 0);
            const int stores = epi(mi, idx) >= 0;
            if (dmas + reads + stores > 1)
                return false;
            if (mi == last && ((read_b_next(mi, idx) >= 0 && idx >= bar) || (read_a_row0(mi, idx) >= 0 && idx < bar)))
                return false;
            if (read_b_next(mi, idx) >= 0) {
                const int b = read_b_blk(mi, idx);
                if (b < 0 || b >= nc || read_b_next(mi, idx) != per_block[b])
                    return false;
                ++per_block[b];
            }
            if (stores) {
                if (epi(mi, idx) != per_row_epi[mi])
                    return false;
                ++per_row_epi[mi];
            }
        }
        for (int b = 0; b < nc; ++b)
            if (per_block[b] != NB)
                return false;
        for (int r = 0; r < last; ++r)
            if (per_row_epi[r] != 5)
                return false;
        for (int p = last * slots + bar; p < rows * slots; ++p)
            if (load_a(p / slots, p % slots) >= 0)
                return false;
        return count(load_a) == la - early && count(load_b) == lb && count(load_a_early) == early &&
               count(read_b_next) == nc * NB && count(read_a_next) == last * NA && count(read_a_row0) == NA &&
               early + 2 * 2 == la;
    }
};
static_assert(PlanSW::check() && PlanSW::vm_at_barrier() == 9 && PlanSW::la == 6 && PlanSW::lb == 9,
              "short-wide slot plan");
static_assert(2 * PlanSW::la * kWaves * 1024 + 3 * PlanSW::lb * kWaves * 1024 <= kLdsBytes,
              "short-wide operand stages fit in LDS");

// ---------------------------------------------------------------------------------------
// Device primitives
// ---------------------------------------------------------------------------------------
template <int N> using ic = std::integral_constant<int, N>;
template <int B, int E, typename F> __device__ __forceinline__ void sfor(F &&f) {
    if constexpr (B < E) {
        f(ic<B>{});
        sfor<B + 1, E>(static_cast<F &&>(f));
    }
}

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Make a value look freshly produced at this point. Values derived from it are then
// recomputed next to their uses inside the loop instead of being hoisted out of it as loop
// invariants (which would keep dozens of precomputed addresses live across the K loop).
__device__ __forceinline__ void fresh_v(int &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void fresh_s(uint32_t &v) { asm volatile("" : "+s"(v)); }
// v ^ X as one VALU instruction (a pure asm statement: the four transposed reads of a fragment
// share it; volatile, one per read, the fp8 wgrad kernel took 3 % longer).
template <int X> __device__ __forceinline__ int xor_here(int v) {
    if constexpr (X == 0) {
        return v;
    } else {
        int r;
        asm("v_xor_b32 %0, %1, %2" : "=v"(r) : "i"(X), "v"(v));
        return r;
    }
}

// Buffer resource for the LDS DMA (SGPR quad): base, stride 0, byte bound, gfx9 raw format.
__device__ __forceinline__ i32x4 dma_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    i32x4 r;
    r[0] = static_cast<int>(static_cast<uint32_t>(a));
    r[1] = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xffffu);
    r[2] = static_cast<int>(bytes);
    r[3] = 0x00020000;
    return r;
}

// 64 lanes x 16 B from global (resource + lane offset + K-step offset) into LDS at
// M0 + 16 * lane. The compiler cannot see this LDS write: waits are placed by hand.
// set_m0 must precede the load by at least one instruction (SALU M0 write -> LDS DMA).
// s_add_u32 writes SCC: the clobber keeps the compiler from holding a branch condition in SCC
// across it.
template <int OFF> __device__ __forceinline__ void set_m0(uint32_t lds_base) {
    asm volatile("s_add_u32 m0, %0, %1" : : "s"(lds_base), "n"(OFF) : "memory", "scc");
}
// A VMEM instruction that reads an SGPR written by a VALU instruction (v_readlane_b32 of a
// spilled SGPR, v_readfirstlane_b32, v_cmp) needs 5 wait states in between. The compiler's
// hazard recognizer does not look inside inline asm, and under SGPR pressure it reloads a DMA's
// soffset with v_readlane_b32 right before it (seen in the fp8 dgrad kernel's first cross-tile
// step: the DMA then used the stale soffset and loaded the wrong K step). The DMAs of the cold
// paths (prologue, a tile's first step, where the spilled values are reloaded) start with 5
// wait states (NOPS = 4); those of the K loop carry none, which costs 4-5 % of throughput, and
// the build checks the generated code for the hazard instead (csrc/check_vmem_sgpr_hazard.py).
template <int NOPS>
__device__ __forceinline__ void dma16_m0(int voff, const i32x4 &rsrc, int soff) {
    if constexpr (NOPS > 0)
        asm volatile("s_nop %3\n\t"
                     "buffer_load_dwordx4 %0, %1, %2 offen " GG_DMA_CPOL " lds"
                     :
                     : "v"(voff), "s"(rsrc), "s"(soff), "n"(NOPS)
                     : "memory");
    else
        asm volatile("buffer_load_dwordx4 %0, %1, %2 offen " GG_DMA_CPOL " lds"
                     :
                     : "v"(voff), "s"(rsrc), "s"(soff)
                     : "memory");
}
__device__ __forceinline__ void dma16(uint32_t lds_dst, int voff, const i32x4 &rsrc, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\t"
                 "s_nop 4\n\t"
                 "buffer_load_dwordx4 %1, %2, %3 offen " GG_DMA_CPOL " lds"
                 :
                 : "s"(lds_dst), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

template <int VM> __device__ __forceinline__ void wait_vm_lds_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

template <bool F16>
__device__ __forceinline__ void mfma(f32x4 &c, const i32x4 &a, const i32x4 &b) {
    if constexpr (F16)
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    else
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// First K half of a tile: C = 0, so the accumulators need no clearing.
template <bool F16>
__device__ __forceinline__ void mfma_first(f32x4 &c, const i32x4 &a, const i32x4 &b) {
    if constexpr (F16)
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
    else
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
}

// fp8 x fp8 -> fp32, 16 x 16 x 128 (gfx950): both sources are 32 bytes of a row per lane.
// The kernel passes w (B) as src0 and x (A) as src1: cbsz gives src0's format, blgp src1's
// (0 e4m3, 1 e5m2).
typedef int i32x8 __attribute__((ext_vector_type(8)));
template <bool BE5, bool AE5, bool FIRST>
__device__ __forceinline__ void mfma8(f32x4 &c, const i32x8 &b, const i32x8 &a) {
#define GG_MFMA8(MODS)                                                                                    \
    if constexpr (FIRST)                                                                                  \
        asm volatile("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, 0" MODS : "=a"(c) : "v"(b), "v"(a));       \
    else                                                                                                  \
        asm volatile("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" MODS : "+a"(c) : "v"(b), "v"(a));
    if constexpr (BE5 && AE5) {
        GG_MFMA8(" cbsz:1 blgp:1")
    } else if constexpr (BE5) {
        GG_MFMA8(" cbsz:1")
    } else if constexpr (AE5) {
        GG_MFMA8(" blgp:1")
    } else {
        GG_MFMA8("")
    }
#undef GG_MFMA8
}

// Four fp32 accumulators -> four 16-bit outputs (RNE), as two packed dwords.
template <bool F16> __device__ __forceinline__ u32x2 pack4(const f32x4 &v) {
    u32x2 r;
    if constexpr (F16) {
        r[0] = __builtin_bit_cast(unsigned, f16x2{(_Float16)v[0], (_Float16)v[1]});
        r[1] = __builtin_bit_cast(unsigned, f16x2{(_Float16)v[2], (_Float16)v[3]});
    } else {
        r[0] = __builtin_bit_cast(unsigned, bf16x2{(__bf16)v[0], (__bf16)v[1]});
        r[1] = __builtin_bit_cast(unsigned, bf16x2{(__bf16)v[2], (__bf16)v[3]});
    }
    return r;
}

// ---------------------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------------------
// Cross-tile pipeline (kernel variant CROSS, for workgroups with several tiles of
// >= kCrossMinSteps K steps): the DMAs of a tile's last three K steps already fetch the first K
// steps of the workgroup's next tile, so a tile boundary has no prologue bubble and no drained
// pipeline. The finished tile's accumulators are stored from registers inside the next tile's
// first step, row block by row block, just before its first MFMAs overwrite them.
#ifndef GG_CROSS_TILE
#define GG_CROSS_TILE 1
#endif
#ifndef GG_STORE_CPOL
#define GG_STORE_CPOL 2 // cache policy of the register-direct C stores: bit 0 sc0, bit 1 nt, bit 4 sc1
#endif
constexpr bool kCrossAllowed  = GG_CROSS_TILE;
constexpr int  kCrossMinSteps = kCrossMinStepsHost; // the three prefetching steps follow the first
constexpr int  kStoreCpol     = GG_STORE_CPOL;
// The ninth column block of short-wide tiles goes out in 32-byte row pieces, the two halves of
// each 64-byte piece from two waves: with the default (write-back) policy the halves meet in L2
// and leave as one write; non-temporal, each half went out on its own and the launch wrote 1.13x
// its output bytes (32 x 520 x 2880 x 2880; 1.00x now, same time).
constexpr int kStoreCpolHalf = 0;
#ifndef GG_PARTIAL_NT
#define GG_PARTIAL_NT 0
#endif
constexpr bool kPartialNt = GG_PARTIAL_NT; // split-K partial sums stored non-temporal (2-5 % slower)


// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int64_t wave_inclusive_sum(int64_t v, int lane) {
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t u = __shfl_up(v, d, 64);
        if (lane >= d)
            v += u;
    }
    return v;
}

// One group of an in-kernel group table: lane g holds group g (g < group_num <= 64).
struct LaneGroup {
    int64_t row0;  // first row (0 for an invalid group)
    int     m;     // rows (0 for an invalid group)
    int     tile0; // first logical tile
    int     tiles; // tiles the group owns
};

// The group table of device-resident sizes for at most 64 groups, one group per lane, by the
// rules of build_group_table_kernel: a negative length, or rows outside [0, total_m), make a
// group invalid (no rows; forward / dgrad: no tiles; wgrad: its out_rows x N tiles, written as
// zeros). Returns the lane's group; *total (uniform) is the tile count, 0 with *overflow set when
// it exceeds 32 bits; *first_bad the first invalid group or -1.
__device__ __forceinline__ LaneGroup lane_group_table(const int64_t *lens, const int64_t *offs, int group_num,
                                                      int64_t total_m, int n_tiles, int out_rows, int lane,
                                                      int *total, int *first_bad, int *overflow) {
    const bool live = lane < group_num;
    int64_t    m    = live ? lens[lane] : 0;
    bool       ok   = m >= 0 && m <= INT32_MAX;
    if (!ok)
        m = 0;
    const int64_t rows_incl = wave_inclusive_sum(m, lane);
    const int64_t row0      = offs != nullptr ? (live ? offs[lane] : 0) : rows_incl - m;
    ok                      = ok && row0 >= 0 && row0 <= total_m && m <= total_m - row0;
    const int64_t tiles     = out_rows > 0 ? (live ? cdiv(out_rows, kTileM) * n_tiles : 0)
                                           : (ok ? cdiv(m, kTileM) * n_tiles : 0);
    const int64_t tiles_incl = wave_inclusive_sum(tiles, lane);
    // the total from lane 63, read into scalar registers (a shuffle would leave it in a VGPR and
    // every value derived from it, the tile loop's bounds included, with it)
    const int64_t all = static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(tiles_incl), 63))) |
                        (static_cast<int64_t>(__builtin_amdgcn_readlane(static_cast<int>(tiles_incl >> 32), 63)) << 32);
    const uint64_t bad = __ballot(live && !ok);
    *first_bad = bad != 0 ? static_cast<int>(__builtin_ctzll(bad)) : -1;
    *overflow  = all > INT32_MAX ? 1 : 0;
    *total     = all > INT32_MAX ? 0 : static_cast<int>(all);
    LaneGroup lg;
    lg.row0  = ok ? row0 : 0;
    lg.m     = ok ? static_cast<int>(m) : 0;
    lg.tile0 = static_cast<int>(min<int64_t>(tiles_incl - tiles, INT32_MAX));
    lg.tiles = static_cast<int>(min<int64_t>(tiles, INT32_MAX));
    return lg;
}

// Cycle stamps (instrumented builds only: `make stamps` compiles the library into lib_stamps/ with
// GG_STAMPS=1; stamps.py reads them). Lane 0 of wave 0 of workgroup w writes the shader clock
// (s_memtime) into slot i of g_stamps[w * kStampSlots ..] with a vector store: 0 kernel start,
// 1 after the prologue, 2 + 5 j .. 6 + 5 j for the workgroup's tile j < 7 (before its first K
// step, after it, after the unchecked steps, after locating the next tile, after the last step),
// 62 before the final LDS epilogue (cross-tile), 63 kernel end; slots 48 and 49 hold the constant
// 100 MHz clock (s_memrealtime, one counter for the whole GPU) at kernel start and end. The stores
// count in vmcnt and only make the hand-placed waits longer.
#ifndef GG_STAMPS
#define GG_STAMPS 0
#endif
constexpr int kStampSlots = 64, kStampWgs = 1024;
#if GG_STAMPS
__device__ unsigned long long g_stamps[kStampWgs * kStampSlots];
#define GG_STAMP(i)                                                                                   \
    do {                                                                                              \
        const unsigned long long t_stamp_ = __builtin_readcyclecounter();                             \
        if (threadIdx.x == 0 && (i) < kStampSlots && blockIdx.x < kStampWgs)                          \
            g_stamps[blockIdx.x * kStampSlots + (i)] = t_stamp_;                                      \
    } while (0)
#define GG_STAMP_REAL(i)                                                                              \
    do {                                                                                              \
        const unsigned long long t_stamp_ = __builtin_amdgcn_s_memrealtime();                         \
        if (threadIdx.x == 0 && blockIdx.x < kStampWgs)                                               \
            g_stamps[blockIdx.x * kStampSlots + (i)] = t_stamp_;                                      \
    } while (0)
#else
#define GG_STAMP(i) \
    do {            \
    } while (0)
#define GG_STAMP_REAL(i) \
    do {                 \
    } while (0)
#endif
constexpr int kStampRealStart = 48, kStampRealEnd = 49;

// Partial tiles: a wave skips the MFMAs of its 16-row blocks that hold no valid output (1), or
// computes every block (0).
#ifndef GG_TAIL_SKIP
#define GG_TAIL_SKIP 1
#endif
constexpr bool kTailSkip = GG_TAIL_SKIP;

// Row-major accumulators (whole-tile 16-bit and fp8 forward, cross-tile): the x fragment
// is the MFMA's first source, so lane l of block (mi, ni) holds output column slot l%16 of rows
// 4 (l/16) .. +3; column slot s of block ni is tile column 8 s + ni of the wave's 128 (the w
// fragment of block ni gathers w rows ni, ni + 8, ..). Over its 8 blocks a lane then holds 8
// consecutive columns of each of its 4 rows: one store is 4 rows x 256 bytes, 4 consecutive
// lanes on 64 contiguous bytes of one row, with no cross-lane moves (0: C^T accumulators, w as
// the first source, and the permlane / DPP line stores). A tail split's K ranges store their fp32
// partial sums as a row-major 256 x 256 slab (tail_reduce_kernel's kCtSlab order).
#ifndef GG_CT
#define GG_CT 1
#endif
constexpr bool ct_instance(int mode, int shape, bool cross) {
    // the 16-bit forward and the fp8 forward (both operands of one format: the MFMA's format
    // modifiers follow the operands when x becomes its first source), 256-column tiles; and the
    // 16-bit forward's short-wide tiles, whose ninth column block keeps C^T accumulators
    return GG_CT && cross &&
           (((mode == make_mode(kFwd, kIn16) || mode == make_mode(kFwd, kInE4M3) || mode == make_mode(kFwd, kInE5M2)) &&
             shape == kShapeWide) ||
            (mode == make_mode(kFwd, kIn16) && shape == kShapeShortWide));
}


// MODE: layout (forward, dgrad, wgrad: operand layouts and tile mapping) and input format.
// CROSS: cross-tile pipeline (needs k_tiles >= kCrossMinSteps); otherwise every tile starts
// with a prologue and ends with the LDS-staged epilogue.
// SHAPE kShapeNarrow (per-tile forward only): tiles of 256 x 224 instead of 256 x 256, for
// one-round problems whose 256-wide tiles leave CUs idle (1 x 2048 x 7168: 224 tiles of 256 x 256,
// 256 of 256 x 224). Each wave takes 7 column blocks (columns 112 wn + 16 ni); the 8th block's
// MFMAs are compiled out, and the memory schedule is unchanged: the B DMAs of rows 224-255 fall
// outside the tile's bounded resource (zeros, no traffic), and the LDS epilogue drops chunks past
// n_valid.
// SHAPE kShapeShort (16-bit forward and dgrad): tiles of args.tile_m <= 192 rows x 256. Each wave takes its
// first 6 interleaved row blocks (tile rows up to 191); the MFMAs, x fragment reads and stores
// of blocks 6 and 7 are compiled out and the memory schedule is unchanged: the A DMAs of rows
// past tile_m fall outside the bounded resource (zeros, no traffic).
// SHAPE kShapeShortWide (cross-tile 16-bit forward): tiles of args.tile_m <= 192 rows x 288. Each
// wave takes 6 interleaved row blocks and 9 column blocks, on its own slot
// plan (PlanSW) with A stages of 192 rows and B stages of 288 rows. With row-major accumulators
// (GG_CT) a wave's columns are 128 wn .. +128 (8 row-major blocks) and 256 + 16 wn .. +16 (the
// ninth block, C^T, stored on its own with 8 bytes per lane); otherwise 144 wn .. +144 and the
// ninth block goes out in the fused stores and as a second pass of the LDS epilogue.
// TAIL (cross-tile 16-bit forward only): the plan cuts its last-round tiles into K ranges (tail
// split: K ranges of last-round tiles store partial sums from epilogue_lds); instances without it
// carry none of its state.
// KT: the problem may have a partial K step (K-major operands mask the chunks past K; MN-major
// ones put the K step in the lane offset, whose range check drops rows past K) or a column tail
// of an MN-major operand (lanes past the stored row masked). Instances with KT = false (the plan
// says there is neither: KernelArgs::tails == 0) give their checked steps the unchecked steps'
// DMA offsets, with no per-DMA VALU OR or add between the offset and the DMA (that cost 2.4 %
// on config 3).
template <bool F16, bool CROSS, int MODE, int SHAPE = kShapeWide, bool TAIL = false, bool KT = true>
__global__ void __launch_bounds__(kThreads, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
grouped_gemm_kernel(const KernelArgs args) {
    constexpr bool A_MN   = mode_a_mn(MODE), B_MN = mode_b_mn(MODE);
    constexpr bool F8     = mode_f8(MODE);
    constexpr int  LAYOUT = mode_layout(MODE);
    constexpr int  ES     = F8 ? 1 : 2;        // input bytes per element
    constexpr int  KS     = kRowBytes / ES;    // contraction values per K step
    // Row blocks of a wave: interleaved (wave wm's block mi is tile rows 16 (2 mi + wm) ..) when A
    // is K-major, so that the valid rows of a partial tile split evenly between the wm = 0 and
    // wm = 1 waves; contiguous (128 wm + 16 mi ..) for the MN-major A of wgrad.
    constexpr bool NARROW = SHAPE == kShapeNarrow;
    constexpr bool SWIDE  = SHAPE == kShapeShortWide;
    constexpr bool SHORT  = SHAPE == kShapeShort || SWIDE; // at most 192 rows per tile
    static_assert(!NARROW || (!CROSS && MODE == make_mode(kFwd, kIn16)), "narrow tiles: per-tile 16-bit forward");
    static_assert(!SHORT || MODE == make_mode(kFwd, kIn16) || MODE == make_mode(kDgrad, kIn16),
                  "short tiles: 16-bit forward and dgrad");
    static_assert(!SWIDE || (CROSS && !TAIL && MODE == make_mode(kFwd, kIn16)),
                  "short-wide tiles: cross-tile 16-bit forward, no tail split");
    constexpr int  TN     = NARROW ? kNarrowTileN : SWIDE ? kShortWideTileN : kTileN; // output columns per tile
    constexpr int  WCOLS  = TN / 2;                          // columns per wave (wn)
    constexpr int  NBLK   = WCOLS / 16;                      // column blocks per wave with MFMAs
    constexpr int  RB     = SHORT ? kShortTileM / 32 : 8;    // row blocks per wave with MFMAs
    constexpr bool ILV    = !A_MN;
    static_assert(!SHORT || ILV, "short tiles: interleaved row blocks");
    constexpr int  A_BLK  = ILV ? 32 : 16; // tile rows between a wave's consecutive row blocks
    // Partial tiles skip their empty row blocks (thin K steps), in every layout, in the cross-tile
    // variant: with one tile per workgroup (the per-tile variant's usual case) the full tiles set
    // the launch time whatever the partial ones save, and the per-tile instances stay smaller.
    constexpr bool kThin  = kTailSkip && CROSS;
    constexpr bool FRONT = GG_PLAN == 1 && !F8 && !SWIDE && !A_MN && !B_MN && RB == 8;
    using P = std::conditional_t<
        F8, Plan8<reads_per_frag(A_MN), reads_per_frag(B_MN)>,
        std::conditional_t<SWIDE, PlanSW,
                           std::conditional_t<FRONT, PlanFront, Plan<reads_per_frag(A_MN), reads_per_frag(B_MN), RB>>>>;
    static_assert(!SWIDE || (NBLK == P::nc && RB == P::rows), "short-wide plan");
    // row-major accumulators (GG_CT): whole 256 x 256 tiles of the 16-bit forward, cross-tile
    constexpr bool CT = ct_instance(MODE, SHAPE, CROSS);
    static_assert(!CT || (RB == 8 && NBLK == 8 && P::nc == 8) || (SWIDE && NBLK == 9 && P::nc == 9),
                  "row-major accumulators: whole tiles, or short-wide tiles (ninth block C^T)");
    constexpr int B_BLK = CT ? 1 : 16; // LDS rows between the w fragments of consecutive column blocks
    constexpr int NC   = P::nc;                                     // column blocks in the registers
    constexpr int A_ST = P::la * kWaves * 1024;                     // bytes of an A stage
    constexpr int B_ST = P::lb * kWaves * 1024;                     // bytes of a B stage
    constexpr int LV   = P::la > P::lb ? P::la : P::lb;             // DMA lane offsets per operand
    // 256-column short tiles keep the 8-DMA A stage of the wide plan; its DMAs j >= 6 cover tile
    // rows 192-255, which a short tile never reads (and which lie outside its resource): not issued
    constexpr auto a_dead = [](int j) { return SHORT && !SWIDE && j * 32 >= kShortTileM; };
    constexpr int CSTR = SWIDE ? kShortWideTileN * 2 + 16 : kCStride; // staged C row stride
    static_assert(kAStages * A_ST + kBStages * B_ST <= kLdsBytes && kShortTileM * CSTR <= kLdsBytes, "LDS");
    static_assert(!(F8 && F16), "fp8 writes bf16");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kLdsBytes];
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8 *)smem));

    const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6) & 3;
    const int wm = wave >> 1, wn = wave & 1;
    const int K = args.k, N = args.n;
    int       T = args.k_tiles; // K steps of the current tile (per group for wgrad)
    // In-kernel group table (device-resident sizes, at most 64 groups): every wave builds it,
    // lane g holding group g; workgroup 0 reports the tile count and the first invalid group.
    // Short tiles and the per-tile fp8 wgrad instances take host-built tables only: the host never
    // plans them with an in-kernel table (a device-size wgrad plan runs cross-tile), and the lane
    // table's registers would push the fp8 wgrad instance with tail masks past 256 VGPRs.
    constexpr bool kLaneTable = !SHORT && !(F8 && !CROSS && LAYOUT == kWgrad);
    const bool     in_kernel_table = kLaneTable && args.d_lens != nullptr;
    LaneGroup  lgrp{0, 0, 0, 0};
    int        lg_total = 0;
    if (in_kernel_table) {
        int first_bad, overflow;
        lgrp = lane_group_table(args.d_lens, args.d_offs, args.group_num, args.lens_rows, args.n_tiles,
                                LAYOUT == kWgrad ? args.m_out : 0, lane, &lg_total, &first_bad, &overflow);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            args.d_header->total_tiles = lg_total;
            args.d_header->first_bad   = first_bad;
            args.d_header->overflow    = overflow;
            args.d_header->reserved    = 0;
        }
    }
    // Tile count: from the kernel arguments, or from a group table built on the device.
    const int total_tiles = in_kernel_table         ? lg_total
                            : args.d_total != nullptr ? __builtin_amdgcn_readfirstlane(*args.d_total)
                                                      : args.total_tiles;
    // Work units: a tile, or with split-K (per-tile variant only) one K range of a tile; unit
    // u = split * total_tiles + tile.
    const int splits      = CROSS ? 1 : args.splits;
    // Tail split (cross-tile variant, host-size plans): the tiles of the last, partial round
    // (rem < half the grid) are cut into tail_s K ranges, one per workgroup, so every workgroup
    // ends the launch after its full rounds plus 1/tail_s of a tile instead of half the grid
    // idling through one more tile. Unit u < full is tile u; u >= full is K range
    // (u - full) / rem of last-round tile (u - full) % rem.
    static_assert(!TAIL || (CROSS && MODE == make_mode(kFwd, kIn16)), "tail split: cross-tile 16-bit forward");
    const int tail_s      = TAIL ? args.tail_splits : 1;
    const int full        = tail_s > 1 ? (total_tiles / static_cast<int>(gridDim.x)) * static_cast<int>(gridDim.x)
                                       : total_tiles;
    const int rem         = total_tiles - full;
    const int total_units = tail_s > 1 ? full + rem * tail_s : total_tiles * splits;

    // DMA lane offsets within a tile's K step (the tile origin is in the buffer resource).
    // K-major operand, row stride ld: DMA j covers tile rows j*32 + wave*8 .. +8; lane -> row
    // lane/8, logical chunk (lane%8) ^ (lane/8).
    // MN-major operand, row stride ld, stored rows = contraction index: DMA j covers
    // contraction rows 4 (2j + wave/2) .. +4 and tile columns 128 (wave%2) .. +128. In LDS the
    // step is 128-byte blocks of 4 rows x 16 columns: block (rb, cb) = (row/4, column/16) sits
    // at byte 128 (16 rb + (cb ^ ((rb / 2) & 1))), so the DMA's 1 KB lands at 1024 (4j + wave)
    // as for a K-major operand; lane -> block column (8 (wave%2) + lane/8) ^ (j & 1), row
    // (lane%8)/2, 8 columns at 8 (lane%2). The column-block swap in every other pair of row
    // blocks puts the blocks that lanes 0-15 and 16-31 of one transposed read take (row blocks
    // rb and rb + 2) in different halves of the 256-byte bank window.
    // fp8 MN-major: in LDS the step is 128 rows of 256 bytes (16 column blocks of 16 columns);
    // LDS row p holds stored row p ^ (16 s), s = (p / 32) & 1, and its 16-byte slot u holds
    // column block 8 ((u / 8) ^ s) + ((u % 8) ^ (p % 8)). DMA j lands at 1024 (4j + wave): LDS
    // rows 16 j + 4 wave + lane/16, slot lane%16, so that 16 lanes read one stored row's 256
    // contiguous bytes (4 consecutive lanes: 64 bytes). The DMA unit takes one cycle per 4-lane
    // group and cache line it touches: 16 per DMA here, against 64 with a lane per stored row.
    // The row swap gives each lane the K order of a K-major fp8 fragment (halves swapped for odd
    // lane/16, see below); the slot permutation spreads the 8 rows of one transposed read over
    // 8 slots, and the half swap puts lanes 0-15 and 16-31 in different halves of the banks.
    const int ld_row   = lane >> 3;
    const int ld_chunk = (lane & 7) ^ ld_row;
    const int mn_c     = (wave & 1) * 8 + (lane >> 3);
    const int f8_rlo   = (4 * wave + (lane >> 4)) & 7; // fp8: LDS row % 8 of the lane's DMA rows
    // column of the lane in a transposed DMA (elements), with column-block swap sw
    auto mn_col = [&](int sw) {
        if constexpr (F8)
            return (8 * (((lane & 15) >> 3) ^ sw) + ((lane & 7) ^ f8_rlo)) * 16;
        else
            return (mn_c ^ sw) * 16 + (lane & 1) * 8;
    };
    // the column-block swap of transposed DMA j
    auto mn_swz = [](int j) { return F8 ? (j >> 1) & 1 : j & 1; };
    // ct: the B operand of row-major accumulators, whose fragments gather rows 8 apart. LDS row p
    // holds stored row p ^ ((p / 8) & 1) (adjacent rows swapped in every other group of 8, so that
    // the 8 rows one read pass gathers alternate between the two halves of the banks) and keeps
    // its chunk c at c ^ (p / 8 % 8). The 8 LDS rows of DMA j share p / 8 = 4 j + wave: lane l
    // fetches stored row 8 (4 j + wave) + ((l / 8) ^ (wave & 1)), logical chunk
    // (l % 8) ^ ((4 j + wave) % 8).
    auto dma_off = [&](bool mn, int j, int ld, bool ct = false) {
        if (ct)
            return (j * 32 + wave * 8 + (ld_row ^ (wave & 1))) * ld * ES + ((lane & 7) ^ ((4 * j + wave) & 7)) * 16;
        if (!mn)
            return (j * 32 + wave * 8 + ld_row) * ld * ES + ld_chunk * 16;
        if (F8)
            return (16 * (j ^ mn_swz(j)) + 4 * wave + (lane >> 4)) * ld + mn_col(mn_swz(j));
        return ((4 * (2 * j + (wave >> 1)) + ((lane & 7) >> 1)) * ld + mn_col(mn_swz(j))) * 2;
    };
    // voff[0]: A's offsets; voff[1]: B's (the forward op shares A's: both row strides are K, and
    // both LDS layouts are the same unless the accumulators are row-major).
    constexpr bool kSameOff = LAYOUT == kFwd && !CT;
    int            voff[kSameOff ? 1 : 2][LV];
    sfor<0, LV>([&](auto j) {
        voff[0][j] = dma_off(A_MN, j, args.lda);
        if constexpr (!kSameOff)
            voff[1][j] = dma_off(B_MN, j, args.ldb, CT && j < 8);
    });
    // MN-major operands in unchecked steps: the lane offsets with the current tile's column mask
    // already applied (set once per tile by set_mn_offsets), and the K step in soffset. Every
    // row of an unchecked step lies inside the contraction, so nothing there relies on the
    // lane offset's range check for rows, and the DMAs need no VALU add and OR per step.
    int voffm[2][kLoads] = {};
    // Last K step when K % 64 != 0: chunks at k >= K get an offset past every bound.
    const int k_last    = K - (T - 1) * KS; // valid K of the last step
    int       ktail_bad = (ld_chunk * (16 / ES) >= k_last) ? static_cast<int>(0x80000000u) : 0;
    // the same for B's DMAs with row-major accumulators, whose logical chunk is (lane % 8) ^
    // ((4 j + wave) % 8): one mask for even DMAs j, one for odd ones
    int ktail_ct[2];
    sfor<0, 2>([&](auto p) {
        const int c  = (lane & 7) ^ ((4 * p + wave) & 7);
        ktail_ct[p] = CT && c * (16 / ES) >= k_last ? static_cast<int>(0x80000000u) : 0;
    });

    // Fragment reads. K-major: lane -> row lane%16 of a 16-row block, logical chunk
    // kh*4 + lane/16 (one base per k-half). MN-major: ds_read_b64_tr_b16 gives lane i of each
    // 16-lane group column i of 4 consecutive rows when source lane s of the group points at
    // row s/4, column 4 (s%4): lane l reads block (row 8 (l/16) + 4 half + 32 kh, column
    // 16 blk) at byte 8 (l%16) of it, i.e. base + 16384 kh + 2048 half + 128 (blk ^ (l/16 & 1));
    // base [blk & 1] holds the lane's part of the swap.
    // ds_read_b128 serves a wave in passes that pair 8-lane groups whose lane/16 differ in bit 0;
    // the fp8 fragment reads chunks 2q and 2q+1 (q = lane/16) in the order kh ^ (q & 1), so that
    // the chunks of such a pair differ in bit 0 as well and take different banks. The lane's K
    // order is then permuted the same way in x and w, which leaves the dot product unchanged.
    // fp8 MN-major: ds_read_b64_tr_b8 gives lane i of each 16-lane group column i of 8 rows when
    // source lane s points at row s/2, column 8 (s%2): read t = 2 kh + half of lane l (q = l/16,
    // s = l%16) takes LDS rows 32 q + 8 t + s/2 (stored rows 32 q + 16 (kh ^ (q & 1)) + 8 half
    // + s/2: the lane's K values in the K-major fragment's order), column block 8 h + blk of
    // the wave's half h, i.e. slot 8 (h ^ (q & 1)) + (blk ^ (s/2)):
    //   (base ^ 16 blk) + 4096 kh + 2048 half,
    //   base = 8192 q + 256 (s/2) + 128 (h ^ (q & 1)) + 16 (s/2) + 8 (s%2),
    // one base per stage (bits 4-6 of it are s/2, so the XOR picks the slot). In one read the
    // 8 rows of a group take 8 different slots, and groups of odd q the other half of the banks.
    const int fr_row = lane & 15, fr_q = lane >> 4;
    const int mn8    = fr_q * 8192 + (fr_row >> 1) * (256 + 16) + (fr_row & 1) * 8;
    int frag_a[2], frag_b[2], frag_bo[2], frag_b8[2]; // frag_bo / frag_b8: row-major accumulators'
                                                      // odd column blocks / short-wide ninth block
    sfor<0, 2>([&](auto kh) {
        const int off = fr_row * kRowBytes +
                        (((F8 ? 2 * fr_q + (kh ^ (fr_q & 1)) : kh * 4 + fr_q) ^ (fr_row & 7)) * 16);
        const int mn  = F8 ? 0 : (lane >> 4) * 4096 + (lane & 15) * 8 + (kh ? -128 : 128) * (fr_q & 1);
        frag_a[kh]    = !A_MN ? wm * (ILV ? 16 : 128) * kRowBytes + off
                        : F8  ? mn8 + 128 * (wm ^ (fr_q & 1))
                              : wm * 1024 + mn;
        // row-major accumulators: lane l reads stored w row 8 (l%16) + ni, at LDS row
        // 8 (l%16) + (ni ^ (l & 1)), whose chunk c sits at c ^ (l%8): block ni adds 128 ni to the
        // base of its parity (frag_b for even ni, frag_bo for odd ni, 256 lower for odd lanes)
        const int ct_off = (8 * fr_row + (fr_row & 1)) * kRowBytes +
                           (((F8 ? 2 * fr_q + (kh ^ (fr_q & 1)) : kh * 4 + fr_q) ^ (fr_row & 7)) * 16);
        frag_bo[kh]   = wn * 128 * kRowBytes + ct_off - (fr_row & 1) * 2 * kRowBytes;
        // short-wide tiles: the ninth block (stored rows 256 + 16 wn + l%16, C^T layout), based so
        // that read_frag's 128 * 8 for block 8 lands on it
        frag_b8[kh]   = (256 + 16 * wn - 8) * kRowBytes + off;
        frag_b[kh]    = CT    ? wn * 128 * kRowBytes + ct_off
                        : !B_MN ? wn * WCOLS * kRowBytes + off
                        : F8  ? mn8 + 128 * (wn ^ (fr_q & 1))
                              : wn * 1024 + mn;
    });

    // Register epilogue: in store s = 2h + half of a 16-row block, lane l writes 16 bytes of
    // row 8 half + l%8 at column ecol + 64 h (see pack_pair). Row-major accumulators: in store
    // s of a 16-row block, lane l writes the 16 bytes of columns ecol .. +7 of row 4 (l/16) + s.
    const int q    = lane >> 4;
    const int ecol = CT ? wn * 128 + 8 * (lane & 15)
                        : wn * (SWIDE ? WCOLS : 128) + ((lane >> 3) & 1) * 32 + (q & 1) * 16 + (q >> 1) * 8;
    int       voffc = CT ? ((wm * 16 + 4 * q) * N + ecol) * 2 : ((wm * (ILV ? 16 : 128) + (lane & 7)) * N + ecol) * 2;
    const int blk_stride = A_BLK * N * 2; // bytes between a wave's 16-row blocks of C

    // Logical stage L of an operand (the K step's index mod 2 for A, mod 3 for B within the
    // tile) lives in physical stage (L + rot) mod n. A tile that follows with prefetched data
    // rotates by its predecessor's K-step count.
    int      rot_a = 0, rot_b = 0;
    int      a_rd[2][2], b_rd[3][2]; // LDS read base per logical stage and k-half
    int      b_rdo[3][2];            // row-major accumulators: B's base for odd column blocks
    int      b_rd8[3][2];            // ... and for a short-wide tile's ninth block
    uint32_t a_dst[2], b_dst[3];     // this wave's DMA destination per logical stage
    auto set_stages = [&]() {
        sfor<0, 2>([&](auto L) {
            const int p = ((L + rot_a) & 1) * A_ST;
            a_dst[L]    = lds0 + wave * 1024 + a_stage(0) + p;
            sfor<0, 2>([&](auto h) { a_rd[L][h] = frag_a[h] + a_stage(0) + p; });
        });
        sfor<0, 3>([&](auto L) {
            int s = L + rot_b;
            s     = s >= 3 ? s - 3 : s;
            const int p = kAStages * A_ST + s * B_ST;
            b_dst[L]    = lds0 + wave * 1024 + p;
            sfor<0, 2>([&](auto h) { b_rd[L][h] = frag_b[h] + p; });
            if constexpr (CT)
                sfor<0, 2>([&](auto h) { b_rdo[L][h] = frag_bo[h] + p; });
            if constexpr (CT && SWIDE)
                sfor<0, 2>([&](auto h) { b_rd8[L][h] = frag_b8[h] + p; });
        });
    };
    // Re-materialise loop-invariant offsets at the top of every loop body (see fresh_v).
    auto refresh = [&]() {
        sfor<0, LV>([&](auto j) {
            fresh_v(voff[0][j]);
            if constexpr (!kSameOff)
                fresh_v(voff[1][j]);
            if constexpr (A_MN)
                fresh_v(voffm[0][j]);
            if constexpr (B_MN)
                fresh_v(voffm[1][j]);
        });
        fresh_v(ktail_bad);
        if constexpr (CT) {
            fresh_v(ktail_ct[0]);
            fresh_v(ktail_ct[1]);
        }
        fresh_v(voffc);
        {
            // the step count, opaque: the checked steps' comparisons with it are made in the loop,
            // not hoisted out of it as lane masks kept in (spilled) SGPRs
            uint32_t t_ = static_cast<uint32_t>(T);
            fresh_s(t_);
            T = static_cast<int>(t_);
        }
        sfor<0, 2>([&](auto L) {
            fresh_s(a_dst[L]);
            sfor<0, 2>([&](auto h) { fresh_v(a_rd[L][h]); });
        });
        sfor<0, 3>([&](auto L) {
            fresh_s(b_dst[L]);
            sfor<0, 2>([&](auto h) { fresh_v(b_rd[L][h]); });
            if constexpr (CT)
                sfor<0, 2>([&](auto h) { fresh_v(b_rdo[L][h]); });
            if constexpr (CT && SWIDE)
                sfor<0, 2>([&](auto h) { fresh_v(b_rd8[L][h]); });
        });
    };
    auto lds_read = [&](int off) -> i32x4 { return *reinterpret_cast<const i32x4 *>(smem + off); };
    typedef short i16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
    auto lds_read_tr = [&](int off) -> u32x2 {
        if constexpr (F8)
            return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2 *)(smem + off)));
        else
            return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(smem + off)));
    };
    // LDS read op r (Plan numbering) of the fragment of 16-row block blk into f (per k-half),
    // from the logical stage whose read bases are rd.
    auto read_frag = [&]<bool MN, int R, int BLK_ROWS = 16>(i32x4(&f)[2], const int(&rd)[2], auto blk) {
        if constexpr (!MN) {
            f[R] = lds_read(rd[R] + blk * BLK_ROWS * kRowBytes);
        } else {
            constexpr int kh = R >> 1, half = R & 1;
            u32x2         v;
            if constexpr (F8)
                v = lds_read_tr(xor_here<16 * decltype(blk)::value>(rd[0]) + kh * 4096 + half * 2048);
            else
                v = lds_read_tr(rd[blk & 1] + kh * 16384 + half * 2048 + blk * 128);
            f[kh][2 * half]     = static_cast<int>(v[0]);
            f[kh][2 * half + 1] = static_cast<int>(v[1]);
        }
    };

    // B's read bases of logical stage L for column block blk (odd blocks of row-major
    // accumulators have their own, see frag_bo)
    auto b_base = [&](int L, auto blk) -> const int(&)[2] {
        if constexpr (CT && decltype(blk)::value == 8)
            return b_rd8[L];
        else if constexpr (CT && (decltype(blk)::value & 1))
            return b_rdo[L];
        else
            return b_rd[L];
    };
    f32x4 acc[8][NC];
    i32x4 fa[2][2];     // x fragments: row ring x k-half
    i32x4 fb[2][NC][2]; // w fragments: step parity x column block x k-half

    // One output tile: its DMA sources and where its C block goes.
    struct Tile {
        i32x4     rsrc_a, rsrc_b; // A / B storage of the tile, bounded to its valid rows
        uint16_t *c_ptr;          // output block origin
        int       m_valid, n_valid;
        int       o0a, o0b;       // MN-major operands: first stored column of the tile
        int       T;              // K steps (wgrad: of the tile's group, at least 1)
        int       k0;             // first K step (split-K: the split's range), 0 otherwise
        int       klast;          // the range ends with the problem's last (maybe partial) K step
        int       tail;           // tail split: index of the last-round tile (-1: a whole tile)
        int       tail_k;         // tail split: the unit's K range (0 .. tail_s - 1)
        float     scale;          // fp8: x scale * w[g] scale (1 otherwise)
        uint32_t  rows;           // this wave's row blocks (bit mi) that hold a valid output
    };
    const int bad_off = static_cast<int>(0x80000000u);
    int       g       = 0; // group hint of locate_tile (a workgroup's logical tiles grow, but
                           // for split-K units, which make_tile restarts the scan for)
    // The group table and the fp8 scales do not change while the kernel runs: read through the
    // constant address space they take scalar loads (lgkmcnt). Through a global pointer the
    // compiler issues vector loads and waits for them with vmcnt(0), which also drains every
    // operand DMA in flight, once per table entry the tile walk reads.
    const const_space<GroupEntry> const_table = to_const_space(args.groups);
    // Tile descriptors (host-size plans of whole tiles, at most 64 per workgroup): lane i holds
    // this workgroup's i-th tile, its first row in x / out, its group and (N-tile << 9 | valid
    // rows); wgrad: the group's first token, its group, (N-tile << 16 | M-tile) and the group's
    // tokens. make_tile reads them with three or four v_readlane instead of walking
    // the XCD remap, the group table and the band order (divisions and dependent scalar loads
    // between the K loops, where no MFMA issues).
    const bool use_desc = !TAIL && splits == 1 && args.desc != nullptr;
    int        d_row0 = 0, d_g = 0, d_tnm = 0, d_m = 0;
    if (use_desc && lane < args.desc_per_wg) {
        const i32x4 dv = reinterpret_cast<const i32x4 *>(args.desc)[static_cast<int>(blockIdx.x) * args.desc_per_wg + lane];
        d_row0         = dv[0];
        d_g            = dv[1];
        d_tnm          = dv[2];
        if constexpr (LAYOUT == kWgrad)
            d_m = dv[3];
    }
    auto      make_tile = [&](int t, int ti) -> Tile {
        // split-K: one unit per workgroup, no L2 sharing across rounds to arrange
        int split = 0, nsplit = splits, L = 0, tail = -1;
        if (use_desc) {
            // the descriptor holds the tile
        } else if (splits > 1) {
            split = t / total_tiles;
            L     = t - split * total_tiles;
            // A workgroup's units wrap around the tile list when units outnumber the grid (the
            // grid is not a multiple of the tile count), so its logical tiles are not monotone:
            // restart the group scan, whose hint only moves forward, when the tile lies before
            // the hinted group.
            if (!in_kernel_table && L < const_table[g].tile0)
                g = 0;
        } else if (TAIL && t >= full) {
            // a K range of a last-round tile: that tile's place in the round decides the XCD order
            tail   = (t - full) % rem;
            split  = (t - full) / rem;
            nsplit = tail_s;
            L      = xcd_remap(full + tail, total_tiles, gridDim.x, args.n_xcd);
        } else {
            L = xcd_remap(t, total_tiles, gridDim.x, args.n_xcd);
        }
        int        tm = 0, tn;
        GroupEntry ge{0, 0, 0};
        int        desc_row0 = 0, desc_mv = 0; // use_desc: the tile's first row and valid rows
        if (use_desc) {
            ti        = __builtin_amdgcn_readfirstlane(ti);
            desc_row0 = __builtin_amdgcn_readlane(d_row0, ti);
            g         = __builtin_amdgcn_readlane(d_g, ti);
            const int tnm = __builtin_amdgcn_readlane(d_tnm, ti);
            if constexpr (LAYOUT == kWgrad) { // the group's first token and size, M- and N-tile
                ge.row0 = desc_row0;
                ge.m    = __builtin_amdgcn_readlane(d_m, ti);
                tm      = tnm & 0xffff;
                tn      = tnm >> 16;
            } else {
                tn      = tnm >> 9;
                desc_mv = tnm & 511;
            }
        } else if (in_kernel_table) {
            // the one lane whose group owns logical tile L
            const uint64_t hit = __ballot(lane < args.group_num && lgrp.tile0 <= L && L - lgrp.tile0 < lgrp.tiles);
            g                  = __builtin_amdgcn_readfirstlane(static_cast<int>(__builtin_ctzll(hit)));
            ge.row0  = static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lgrp.row0), g))) |
                      (static_cast<int64_t>(__builtin_amdgcn_readlane(static_cast<int>(lgrp.row0 >> 32), g)) << 32);
            ge.m     = __builtin_amdgcn_readlane(lgrp.m, g);
            ge.tile0 = __builtin_amdgcn_readlane(lgrp.tile0, g);
            const int m_tiles = ((LAYOUT == kWgrad ? args.m_out : ge.m) + kTileM - 1) / kTileM;
            band_coords(L - ge.tile0, m_tiles, args.n_tiles, args.band, &tm, &tn);
        } else {
            locate_tile(L, const_table, args.group_num, args.n_tiles, args.band, &g, &tm, &tn,
                        LAYOUT == kWgrad ? args.m_out : 0, SHORT ? args.tile_m : kTileM);
            ge.row0  = const_table[g].row0;
            ge.m     = const_table[g].m;
            ge.tile0 = const_table[g].tile0;
        }
        const uint8_t   *xa = static_cast<const uint8_t *>(args.x); // A storage (bytes)
        const uint8_t   *wb = static_cast<const uint8_t *>(args.w); // B storage (bytes)
        Tile             tl;
        tl.n_valid         = min(TN, N - tn * TN);
        const int64_t col0 = static_cast<int64_t>(tn) * TN;
        tl.o0a = tl.o0b = 0;
        // K range of the unit: steps [k0, k1) of k_tiles, balanced over the splits
        const int k0 = split * args.k_tiles / nsplit, k1 = (split + 1) * args.k_tiles / nsplit;
        tl.T      = k1 - k0;
        tl.k0     = k0;
        tl.klast  = k1 == args.k_tiles;
        tl.tail   = tail;
        tl.tail_k = split;
        tl.scale  = 1.0f;
        if constexpr (LAYOUT == kWgrad) {
            // A^T = grad_out rows of the group, columns tm*256..; B^T = x rows, columns tn*256..
            const int64_t o0a = static_cast<int64_t>(tm) * kTileM;
            const int64_t ma  = static_cast<int64_t>(ge.m) * args.lda - o0a; // elements
            const int64_t mb  = static_cast<int64_t>(ge.m) * args.ldb - col0;
            tl.m_valid = min(kTileM, args.m_out - tm * kTileM);
            tl.rsrc_a  = dma_rsrc(xa + (ge.row0 * args.lda + o0a) * ES, static_cast<uint32_t>(ma > 0 ? ma * ES : 0));
            tl.rsrc_b  = dma_rsrc(wb + (ge.row0 * args.ldb + col0) * ES, static_cast<uint32_t>(mb > 0 ? mb * ES : 0));
            tl.o0a     = static_cast<int>(o0a);
            tl.o0b     = static_cast<int>(col0);
            tl.c_ptr   = static_cast<uint16_t *>(args.out) +
                       (static_cast<int64_t>(g) * args.m_out + o0a) * N + col0;
            // at least the cross-tile pipeline's kCrossMinSteps: the steps past the group's rows
            // read zeros (rows past ge.m fall outside rsrc_a / rsrc_b), so a short or empty group
            // costs a few zero steps instead of the whole launch's cross-tile variant
            tl.T     = max(CROSS ? kCrossMinSteps : 1, static_cast<int>(cdiv(ge.m, KS)));
            tl.k0    = 0;
            tl.klast = 1;
        } else {
            const int TM       = SHORT ? args.tile_m : kTileM; // rows per tile
            tl.m_valid         = use_desc ? desc_mv : min(TM, ge.m - tm * TM);
            const int64_t row0 = use_desc ? static_cast<int64_t>(desc_row0) : ge.row0 + static_cast<int64_t>(tm) * TM;
            tl.rsrc_a = dma_rsrc(xa + row0 * args.lda * ES, static_cast<uint32_t>(tl.m_valid) * args.lda * ES);
            if constexpr (LAYOUT == kFwd) {
                tl.rsrc_b = dma_rsrc(wb + (static_cast<int64_t>(g) * N + col0) * args.ldb * ES,
                                     static_cast<uint32_t>(tl.n_valid) * args.ldb * ES);
            } else {
                // w[g] stored K x N: columns col0.. of all K rows (the end of w[g] bounds it)
                const int64_t per_g = static_cast<int64_t>(K) * args.ldb;
                tl.rsrc_b = dma_rsrc(wb + (g * per_g + col0) * ES, static_cast<uint32_t>((per_g - col0) * ES));
                tl.o0b = static_cast<int>(col0);
            }
            tl.c_ptr = static_cast<uint16_t *>(args.out) + row0 * N + col0;
        }
        if constexpr (F8)
            tl.scale = to_const_space(args.x_scale)[0] * to_const_space(args.w_scale)[g];
        // a short-wide wave with row-major accumulators owns columns 128 wn .. +128 and 256 + 16 wn ..
        // +16: it holds a valid column iff 128 wn < n_valid, as for 256-column tiles
        tl.rows = __builtin_amdgcn_readfirstlane(active_rows(ILV, tl.m_valid, tl.n_valid, wm, wn, SWIDE && !CT ? WCOLS : 128));
        return tl;
    };
    auto c_rsrc = [&](const Tile &tl) {
        // rows past m_valid fall outside the resource
        return __builtin_amdgcn_make_buffer_rsrc(tl.c_ptr, static_cast<short>(0),
                                                 static_cast<int>(tl.m_valid * N * 2), 0x00020000);
    };
    // zero length: no traffic, the DMA writes zeros (all-constant, so no SGPRs held for it)
    const i32x4 rsrc_0 = dma_rsrc(nullptr, 0);

    int t = blockIdx.x;
    if (t >= total_units)
        return;
    GG_STAMP(0);
    GG_STAMP_REAL(kStampRealStart);
    [[maybe_unused]] int stamp_tile = 0; // GG_STAMPS: tiles of this workgroup so far
    int  tile_i = 0; // this workgroup's tile count so far (unit t = blockIdx.x + tile_i * grid)
    Tile cur = make_tile(t, 0), nxt = cur;
    if (!CROSS || LAYOUT == kWgrad || TAIL)
        T = __builtin_amdgcn_readfirstlane(cur.T);
    bool cross_next = false; // the DMAs past this tile's last K step fetch `nxt`

    // Where the DMAs of K step kidx of an operand (false: x, true: w) read from: resource,
    // K offset and the per-lane mask of a partial last step. Unchecked: kidx is a full step of
    // the current tile. Checked: kidx may be the tile's partial last step or lie past it (the
    // next tile's first steps, or nothing). Evaluated once per step and operand stream.
    // MN-major operands: a K step is 64 stored rows, added to the lane offset (not soffset)
    // so that rows past the contraction length fall outside the resource; lane columns past
    // the row get an out-of-range offset (mask). K-major: the K step is soffset, and the
    // partial last step's chunks past K get the out-of-range offset.
    struct DmaSrc {
        i32x4 rs;
        int   so, vadd, mask, mask1; // MN-major: mask for even / odd DMA j (column-block swap)
        int   mask8;                 // B's DMA 8 of short-wide row-major tiles (C^T rows)
    };
    auto dma_src = [&](auto b_op, int kidx, auto checked) -> DmaSrc {
        constexpr bool B  = decltype(b_op)::value;
        constexpr bool MN = B ? B_MN : A_MN;
        const int      ld = B ? args.ldb : args.lda;
        i32x4          rc = cur.rsrc_a, rn = nxt.rsrc_a;
        int            oc = cur.o0a, on = nxt.o0a;
        if constexpr (B) {
            rc = cur.rsrc_b;
            rn = nxt.rsrc_b;
            oc = cur.o0b;
            on = nxt.o0b;
        }
        DmaSrc d;
        if constexpr (decltype(checked)::value) {
            const bool in_cur = kidx < T;
            const int  koff   = in_cur ? kidx : kidx - T;
            // step of the operand: the unit's first step plus koff (the next unit starts at 0 but for
            // a tail split's later K ranges)
            int kabs;
            if constexpr (TAIL)
                kabs = koff + (in_cur ? cur.k0 : nxt.k0);
            else
                kabs = in_cur ? koff + cur.k0 : koff;
            d.rs           = in_cur ? rc : (cross_next ? rn : rsrc_0);
            if constexpr (MN && !KT) { // no partial K step, no column tail
                d.so    = kabs * kTileK * ld * 2;
                d.vadd  = 0;
                d.mask  = 0;
                d.mask1 = 0;
            } else if constexpr (MN) {
                d.so   = 0;
                d.vadd = kabs * kTileK * ld * 2;
                d.mask  = (in_cur ? oc : on) + mn_col(0) >= ld ? bad_off : 0;
                d.mask1 = (in_cur ? oc : on) + mn_col(1) >= ld ? bad_off : 0;
            } else {
                d.so   = kabs * kRowBytes;
                d.vadd = 0;
                // the unit's partial last K step (a next unit has at least kCrossMinSteps steps, so
                // the three prefetched never include its last, and koff < 3 < T - 1 for them)
                const bool tail_step = KT && koff == T - 1 && cur.klast;
                d.mask  = tail_step ? (B && CT ? ktail_ct[0] : ktail_bad) : 0;
                d.mask1 = tail_step && B && CT ? ktail_ct[1] : 0; // odd DMAs of B (row-major acc.)
                d.mask8 = tail_step ? ktail_bad : 0;
            }
        } else {
            d.rs = rc;
            if constexpr (MN) {
                // the column masks are in voffm (set_mn_offsets)
                d.so    = (kidx + cur.k0) * kTileK * ld * 2;
                d.vadd  = 0;
                d.mask  = 0;
                d.mask1 = 0;
            } else {
                d.so   = (kidx + cur.k0) * kRowBytes;
                d.vadd = 0;
                d.mask = 0;
            }
        }
        return d;
    };
    // Lane offset of DMA j of operand b_op for source d.
    auto dma_voff = [&](auto b_op, auto j, const DmaSrc &d, auto checked) -> int {
        constexpr bool B  = decltype(b_op)::value;
        constexpr bool MN = B ? B_MN : A_MN;
        const int      vo = voff[(B && !kSameOff) ? 1 : 0][j];
        if constexpr (MN && !decltype(checked)::value)
            return voffm[B ? 1 : 0][j];
        else if constexpr (MN && !KT)
            return vo;
        else if constexpr (MN)
            return (vo + d.vadd) | (mn_swz(j) ? d.mask1 : d.mask);
        else if constexpr (decltype(checked)::value)
            return vo | ((B && CT && j == 8) ? d.mask8 : (B && CT && (j & 1)) ? d.mask1 : d.mask);
        else
            return vo;
    };
    // The current tile's column masks folded into the MN-major lane offsets (voffm), once per
    // tile before its unchecked steps: the mask of DMA j is that of its column-block swap.
    auto set_mn_offsets = [&](const Tile &tl) {
        sfor<0, kLoads>([&](auto j) {
            if constexpr (A_MN)
                voffm[0][j] = voff[0][j] | (tl.o0a + mn_col(mn_swz(j)) >= args.lda ? bad_off : 0);
            if constexpr (B_MN)
                voffm[1][j] = voff[kSameOff ? 0 : 1][j] | (tl.o0b + mn_col(mn_swz(j)) >= args.ldb ? bad_off : 0);
        });
    };
    // DMA with its own M0 write (prologue).
    auto dma_now = [&](uint32_t dst, auto b_op, auto j, int kidx) {
        sched_fence();
        const DmaSrc d = dma_src(b_op, kidx, std::true_type{});
        dma16(dst + j * 4096, dma_voff(b_op, j, d, std::true_type{}), d.rs, d.so);
        sched_fence();
    };
    // DMA whose M0 was written before the slot's MFMA; cold: with the SGPR wait states.
    auto dma_go = [&](auto b_op, const DmaSrc &d, auto j, auto checked, auto cold) {
        sched_fence();
        dma16_m0<decltype(cold)::value ? 4 : 0>(dma_voff(b_op, j, d, checked), d.rs, d.so);
        sched_fence();
    };
    using A_OP = std::false_type;
    using B_OP = std::true_type;

    // ---- prologue of a tile that starts cold: A(0), B(0..2), the first DMAs of A(1) ----------
    auto issue_prologue = [&]() {
        refresh();
        sfor<0, P::la>([&](auto j) {
            if constexpr (!a_dead(j))
                dma_now(a_dst[0], A_OP{}, j, 0);
        });
        sfor<0, P::lb>([&](auto j) { dma_now(b_dst[0], B_OP{}, j, 0); });
        sfor<0, P::lb>([&](auto j) { dma_now(b_dst[1], B_OP{}, j, 1); });
        sfor<0, P::lb>([&](auto j) { dma_now(b_dst[2], B_OP{}, j, 2); });
        sfor<0, P::early>([&](auto j) { dma_now(a_dst[1], A_OP{}, j, 1); });
    };
    // Then B(0) and A(0) row 0 into registers. VM: DMAs/stores issued after B(1)'s last.
    auto finish_prologue = [&]<int VM>() {
        wait_vm_lds_barrier<VM>(); // A(0), B(0), B(1) landed everywhere
        sfor<0, NC>([&](auto ni) {
            sfor<0, reads_per_frag(B_MN)>([&](auto r) {
                read_frag.template operator()<B_MN, r, B_BLK>(fb[0][ni], b_base(0, ni), ni);
            });
        });
        sfor<0, reads_per_frag(A_MN)>([&](auto r) {
            read_frag.template operator()<A_MN, r, A_BLK>(fa[0], a_rd[0], ic<0>{});
        });
        wait_vm_lds_barrier<63>(); // every wave holds B(0): its stage may be refilled
    };

    // ---- register epilogue: 1 KB stores of 8 rows x 128 B (whole cache lines) ----------------
    // Lane l holds C^T blocks: row l%16, columns 4q..4q+3 of each 16 x 16 block (q = l/16).
    // One v_permlane16_swap per dword between blocks 2j and 2j+1 gives chunk X_j: every lane
    // holds 8 consecutive columns of its row, q = 0, 2 from block 2j, q = 1, 3 from block 2j+1,
    // columns 0-7 (q < 2) or 8-15; 4 lanes cover 64 bytes of a row. Two DPP row shifts then
    // pair X_2h with X_2h+1 so that a store covers whole 128-byte rows:
    //   Z_A: lanes l%16 < 8 keep X_2h (row l%16), lanes l%16 >= 8 take X_2h+1 of lane l-8;
    //   Z_B: lanes l%16 >= 8 keep X_2h+1 (row l%16), lanes l%16 < 8 take X_2h of lane l+8.
    // Z_A holds rows 0-7 and Z_B rows 8-15 of the block, columns 64h..64h+63.
    float prev_scale = 1.0f; // fp8: scale of the tile whose accumulators the fused stores take
    auto  pack_vals = [&](f32x4 v0, f32x4 v1) -> u32x4 { // blocks 2j and 2j+1 -> chunk X_j
        const u32x2 p0 = pack4<F16>(v0);
        const u32x2 p1 = pack4<F16>(v1);
        const auto  s0 = __builtin_amdgcn_permlane16_swap(p0[0], p1[0], false, false);
        const auto  s1 = __builtin_amdgcn_permlane16_swap(p0[1], p1[1], false, false);
        return u32x4{s0[0], s1[0], s0[1], s1[1]};
    };
    auto pack_chunk = [&](auto r, auto j) -> u32x4 {
        // reads of these accumulators may not move above this point
        asm volatile("" : "+a"(acc[r][2 * j]), "+a"(acc[r][2 * j + 1]));
        f32x4 v0 = acc[r][2 * j], v1 = acc[r][2 * j + 1];
        if constexpr (F8) {
            v0 *= prev_scale;
            v1 *= prev_scale;
        }
        return pack_vals(v0, v1);
    };
    auto dpp_pair = [&](const u32x4 &x0, const u32x4 &x1, u32x4 &za, u32x4 &zb) {
        sfor<0, 4>([&](auto i) {
            // row_shr:8 into banks 2-3, row_shl:8 into banks 0-1
            za[int(i)] = __builtin_amdgcn_update_dpp(x0[int(i)], x1[int(i)], 0x118, 0xf, 0xc, false);
            zb[int(i)] = __builtin_amdgcn_update_dpp(x1[int(i)], x0[int(i)], 0x108, 0xf, 0x3, false);
        });
    };
    auto pack_pair = [&](auto r, auto h, u32x4 &za, u32x4 &zb) {
        dpp_pair(pack_chunk(r, ic<2 * h>{}), pack_chunk(r, ic<2 * h + 1>{}), za, zb);
    };
    // Store s = 2h + half of row block r. Chunks past n_valid get an out-of-range offset
    // (N % 8 == 0, so a 16-byte chunk is either all valid or all past N).
    auto store_line = [&](const u32x4 &d, int r, int s_, const __amdgpu_buffer_rsrc_t &crs,
                          int n_valid) {
        const int h  = s_ >> 1, half = s_ & 1;
        // The row block's byte offset from an opaque copy of the stride: computed here (two SALU)
        // instead of 32 loop-invariant offsets that the compiler would keep in (spilled) SGPRs.
        uint32_t bs = static_cast<uint32_t>(blk_stride);
        fresh_s(bs);
        const int vo = ecol + 64 * h < n_valid
                           ? voffc + r * static_cast<int>(bs) + half * (8 * N * 2) + h * 128
                           : static_cast<int>(0x80000000u);
        __builtin_amdgcn_raw_buffer_store_b128(d, crs, vo, 0, kStoreCpol);
    };
    // ---- epilogue through LDS: accumulators -> 16-bit -> LDS (528-byte row stride) -> every wave
    // streams 64 whole rows, two 512-byte rows per 16-byte-per-lane store. Needs all of LDS.
    // Accumulators are only ever written by the MFMAs (inline asm, "+a"): code that assigns them
    // from VGPR values lets the register allocator keep an accumulator in VGPRs across the K loop
    // and copy it around the MFMAs, reading an MFMA's result one wait state after issue.
    // Staging offset of a lane's 4 outputs of block (mi, ni) in the 528-byte-stride C tile.
    auto stage_off = [&]() {
        int row = wm * (ILV ? 16 : 128) + (lane & 15);
        fresh_v(row);
        const int col = wn * WCOLS + (lane >> 4) * 4;
        return row * CSTR + col * 2;
    };
    auto stage_block = [&](const Tile &tl, int off, auto mi, auto ni, f32x4 v) {
        if constexpr (F8)
            v *= tl.scale;
        *reinterpret_cast<u32x2 *>(smem + off + mi * A_BLK * CSTR + ni * 16 * 2) = pack4<F16>(v);
    };
    // Second half of the LDS epilogue: the staged tile to global memory.
    auto store_staged = [&](const Tile &tl) {
        wait_vm_lds_barrier<63>();
        int row = wave * 64 + (lane >> 5);
        fresh_v(row);
        const int chunk = lane & 31;
        const int loff  = row * CSTR + chunk * 16;
        const int goff  = chunk * 8 < tl.n_valid ? (row * N + chunk * 8) * 2 : static_cast<int>(0x80000000u);
        const __amdgpu_buffer_rsrc_t crs = c_rsrc(tl);
        sfor<0, 2>([&](auto half) {
            i32x4 d[16];
            sfor<0, 16>([&](auto i) { d[i] = lds_read(loff + (half * 16 + i) * 2 * CSTR); });
            sfor<0, 16>([&](auto i) {
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, d[i]), crs,
                    goff + (half * 16 + i) * 2 * N * 2, 0, /*nt*/ 2);
            });
        });
        if constexpr (SWIDE) {
            // columns 256-287: four 16-byte chunks per row, 16 rows per store, rows 48 wave .. +48
            int row2 = wave * 48 + (lane >> 2);
            fresh_v(row2);
            const int chunk2 = 32 + (lane & 3);
            const int goff2  = chunk2 * 8 < tl.n_valid ? (row2 * N + chunk2 * 8) * 2 : static_cast<int>(0x80000000u);
            i32x4     d2[3];
            sfor<0, 3>([&](auto i) { d2[i] = lds_read((row2 + 16 * i) * CSTR + chunk2 * 16); });
            sfor<0, 3>([&](auto i) {
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, d2[i]), crs,
                    goff2 + 16 * i * N * 2, 0, /*nt*/ 2);
            });
        }
        wait_vm_lds_barrier<63>(); // every wave is done reading the staged C
    };
    // TAIL: a K range of a last-round tile leaves through here too, as fp32 partial sums (slab
    // k * rem + tail of the workspace, store_partial's register order) for tail_reduce_kernel, the
    // next launch on the stream. One exit path reads the accumulators, branch-free: a whole tile's
    // partial-sum stores go to a zero-length resource and a K range's C stores to a zero-row tile
    // (both dropped). With a second exit path reading them, the register allocator homed an
    // accumulator in VGPRs for the whole kernel and read it back one wait state after its MFMAs
    // (csrc/check_mfma_acc_hazard.py rejects such builds).
    auto epilogue_lds = [&](Tile tl) {
        wait_vm_lds_barrier<0>(); // trailing DMAs landed, every wave is done reading LDS
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory"); // MFMA -> VALU read distance
        const int off = stage_off();
        const bool part = TAIL && tl.tail >= 0;
        const __amdgpu_buffer_rsrc_t prs =
            __builtin_amdgcn_make_buffer_rsrc(args.ws, static_cast<short>(0), part ? 0x7fffffff : 0, 0x00020000);
        const int poff = part ? ((tl.tail_k * rem + tl.tail) * 65536 + wave * 16384 + lane * 4) * 4 : 0;
        if constexpr (TAIL)
            tl.m_valid = part ? 0 : tl.m_valid; // no C rows for a K range
        sfor<0, RB>([&](auto mi) { // short tiles: blocks 6 and 7 are past the tile
            sfor<0, NBLK>([&](auto ni) { // narrow tiles: the 8th block is another wave's columns
                asm volatile("" : "+a"(acc[mi][ni]));
                const f32x4 v = acc[mi][ni];
                if constexpr (TAIL)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                           poff + (mi * 8 + ni) * 1024, 0, 0);
                stage_block(tl, off, mi, ni, v);
            });
        });
        store_staged(tl);
    };
    // ---- split-K unit: its fp32 accumulators to the workspace slab of unit u (256 KB), in
    // register order: wave w, block (mi, ni), lane l at float 65536 u + 16384 w + 256 (8 mi + ni)
    // + 4 l (whole 1 KB per store instruction). split_reduce_kernel adds the slabs of a tile.
    auto store_partial = [&](int u) {
        wait_vm_lds_barrier<0>(); // trailing DMAs landed, every wave is done reading LDS
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory"); // MFMA -> VALU read distance
        float *dst = args.ws + static_cast<int64_t>(u) * 65536 + wave * 16384 + lane * 4;
        sfor<0, 8>([&](auto mi) {
            sfor<0, 8>([&](auto ni) {
                asm volatile("" : "+a"(acc[mi][ni]));
                f32x4 *d = reinterpret_cast<f32x4 *>(dst + (mi * 8 + ni) * 256);
                if constexpr (kPartialNt)
                    __builtin_nontemporal_store(acc[mi][ni], d);
                else
                    *d = acc[mi][ni];
            });
        });
    };

    // ---- one K step ---------------------------------------------------------------------------
    // SA = kt % 2 (A logical stage, w register set), SB = kt % 3 (B logical stage).
    // FUSE: first step of a tile whose predecessor's accumulators are still to be stored (row
    // blocks 1-7 here; block 0 before the step), to prev_crs / prev_n. Nothing to store before
    // the first tile: zero-length resource, the stores are dropped.
    const __amdgpu_buffer_rsrc_t null_crs =
        __builtin_amdgcn_make_buffer_rsrc(nullptr, static_cast<short>(0), 0, 0x00020000);
    __amdgpu_buffer_rsrc_t prev_crs = null_crs;
    int                    prev_n   = 0;
    u32x4                  pair[2];
    // Short-wide tiles: the ninth column block of row block r (columns 144 wn + 128 ..), lane l
    // writing the 8 bytes it holds (row l%16, columns 4 (l/16) ..) of 16 rows x 32 bytes.
    auto store_block9 = [&](auto r, const __amdgpu_buffer_rsrc_t &crs, int n_valid) {
        asm volatile("" : "+a"(acc[r][NC - 1]));
        f32x4 v = acc[r][NC - 1];
        if constexpr (F8)
            v *= prev_scale;
        const int col = (CT ? 256 + 16 * wn : wn * WCOLS + 128) + (lane >> 4) * 4;
        uint32_t  bs  = static_cast<uint32_t>(blk_stride);
        fresh_s(bs);
        const int vo = col < n_valid ? ((wm * 16 + (lane & 15)) * N + col) * 2 + r * static_cast<int>(bs)
                                     : static_cast<int>(0x80000000u);
        __builtin_amdgcn_raw_buffer_store_b64(pack4<F16>(v), crs, vo, 0, kStoreCpolHalf);
    };
    // Row-major accumulators: store s (0-3) of row block r, lane l writing row 4 (l/16) + s of
    // the block at columns ecol .. +7, element s of its 8 column blocks' accumulators (column slot
    // l%16 of block ni is column 8 (l%16) + ni). Columns past n_valid get an out-of-range offset
    // (N % 8 == 0: a 16-byte chunk is all valid or all past N); rows past m_valid fall outside crs.
    // fp8: scaled by the tile's x scale * w[g] scale (`scale`) before the conversion.
    auto store_ct = [&](auto r, auto s_, const __amdgpu_buffer_rsrc_t &crs, int n_valid, float scale) {
        u32x4 d;
        sfor<0, 4>([&](auto u) {
            // reads of these accumulators may not move above this point
            asm volatile("" : "+a"(acc[r][2 * u]), "+a"(acc[r][2 * u + 1]));
            float v0 = acc[r][2 * u][int(s_)], v1 = acc[r][2 * u + 1][int(s_)];
            if constexpr (F8) {
                v0 *= scale;
                v1 *= scale;
            }
            if constexpr (F16)
                d[int(u)] = __builtin_bit_cast(unsigned, f16x2{(_Float16)v0, (_Float16)v1});
            else
                d[int(u)] = __builtin_bit_cast(unsigned, bf16x2{(__bf16)v0, (__bf16)v1});
        });
        // offsets from opaque copies of the strides (two SALU), not loop-invariant ones the
        // compiler would keep in (spilled) SGPRs
        uint32_t bs = static_cast<uint32_t>(blk_stride), rs = static_cast<uint32_t>(N * 2);
        fresh_s(bs);
        fresh_s(rs);
        const int vo = ecol < n_valid ? voffc + r * static_cast<int>(bs) + s_ * static_cast<int>(rs)
                                      : static_cast<int>(0x80000000u);
        __builtin_amdgcn_raw_buffer_store_b128(d, crs, vo, 0, kStoreCpol);
    };
    // Store s (0-3) of the previous tile's row block r: packed with the next one for even s;
    // s = 4 (short-wide tiles): the ninth column block.
    constexpr int kEpiStores = SWIDE ? 5 : 4;
    auto epi_store = [&](auto r, auto s_) {
        sched_fence();
        if constexpr (CT && s_ < 4) {
            store_ct(r, s_, prev_crs, prev_n, prev_scale);
        } else if constexpr (s_ == 4) {
            store_block9(r, prev_crs, prev_n);
        } else {
            if constexpr (s_ % 2 == 0)
                pack_pair(r, ic<s_ / 2>{}, pair[0], pair[1]);
            store_line(pair[s_ % 2], r, s_, prev_crs, prev_n);
        }
        sched_fence();
    };
    // MFMA idx of row mi of a K step (w register set SA; FIRST: the tile's first step, C = 0).
    auto row_mfma = [&]<int SA, bool FIRST>(auto mi_, auto idx_) {
        constexpr int mi = decltype(mi_)::value, idx = decltype(idx_)::value;
        constexpr int kh = idx / P::nc, ni = idx % P::nc; // fp8: one MFMA per (mi, ni), kh = 0
        if constexpr (ni >= NBLK || mi >= RB) {
            // narrow tiles: no 8th column block; short tiles: no row blocks 6 and 7
        } else if constexpr (F8) {
            const i32x8 bw = __builtin_shufflevector(fb[SA][ni][0], fb[SA][ni][1], 0, 1, 2, 3, 4, 5, 6, 7);
            const i32x8 ax = __builtin_shufflevector(fa[mi & 1][0], fa[mi & 1][1], 0, 1, 2, 3, 4, 5, 6, 7);
            if constexpr (CT) // row-major accumulators: x is the first source (cbsz: x's format)
                mfma8<mode_a_e5(MODE), mode_b_e5(MODE), FIRST>(acc[mi][ni], ax, bw);
            else
                mfma8<mode_b_e5(MODE), mode_a_e5(MODE), FIRST>(acc[mi][ni], bw, ax);
        } else if constexpr (CT && ni < 8 && FIRST && kh == 0) // row-major accumulators: x is the first source
            mfma_first<F16>(acc[mi][ni], fa[mi & 1][0], fb[SA][ni][0]);
        else if constexpr (CT && ni < 8)
            mfma<F16>(acc[mi][ni], fa[mi & 1][kh], fb[SA][ni][kh]);
        else if constexpr (FIRST && kh == 0)
            mfma_first<F16>(acc[mi][ni], fb[SA][ni][0], fa[mi & 1][0]);
        else
            mfma<F16>(acc[mi][ni], fb[SA][ni][kh], fa[mi & 1][kh]);
    };
    auto step = [&]<int SA, int SB, bool FIRST, bool CHECKED, bool FUSE>(int kt) {
        // kt is uniform; saying so keeps the checked tail's comparisons and resource selects
        // scalar when the compiler would otherwise carry kt through a branch merge in a VGPR.
        kt = __builtin_amdgcn_readfirstlane(kt);
        constexpr int NX = SA ^ 1;
        constexpr int SB_NEXT = (SB + 1) % 3;
        using chk = std::integral_constant<bool, CHECKED>;
        const DmaSrc src_a1 = dma_src(A_OP{}, kt + 1, chk{}); // A(kt+1)
        const DmaSrc src_b3 = dma_src(B_OP{}, kt + 3, chk{}); // B(kt+3)
        const DmaSrc src_a2 = dma_src(A_OP{}, kt + 2, chk{}); // A(kt+2)
        sfor<0, P::rows>([&](auto mi_) {
            constexpr int mi = decltype(mi_)::value;
            sfor<0, P::slots>([&](auto idx_) {
                constexpr int idx = decltype(idx_)::value;
                constexpr int dj = P::dma_j(mi, idx);
                constexpr int dk = P::dma_kind(mi, idx) == 1 && a_dead(dj) ? 0 : P::dma_kind(mi, idx);
                if constexpr (dk == 1)
                    set_m0<dj * 4096>(a_dst[NX]); // the MFMA below is the wait state
                else if constexpr (dk == 2)
                    set_m0<dj * 4096>(b_dst[SB]);
                else if constexpr (dk == 3)
                    set_m0<dj * 4096>(a_dst[SA]);
                sched_fence();
                row_mfma.template operator()<SA, FIRST>(mi_, idx_);
                sched_fence();
                if constexpr (mi == P::last && idx == P::bar) {
                    wait_vm_lds_barrier<P::vm_at_barrier()>();
                    sched_fence();
                }
                if constexpr (P::read_a_next(mi, idx) >= 0 && mi + 1 < RB) {
                    read_frag.template operator()<A_MN, P::read_a_next(mi, idx), A_BLK>(fa[(mi + 1) & 1], a_rd[SA],
                                                                                 ic<mi + 1>{});
                    sched_fence();
                }
                if constexpr (P::read_b_next(mi, idx) >= 0) {
                    constexpr int bb = P::read_b_blk(mi, idx);
                    read_frag.template operator()<B_MN, P::read_b_next(mi, idx), B_BLK>(fb[NX][bb], b_base(SB_NEXT, ic<bb>{}),
                                                                                 ic<bb>{});
                    sched_fence();
                }
                if constexpr (P::read_a_row0(mi, idx) >= 0) {
                    read_frag.template operator()<A_MN, P::read_a_row0(mi, idx), A_BLK>(fa[0], a_rd[NX], ic<0>{});
                    sched_fence();
                }
                if constexpr (FUSE && P::epi(mi, idx) >= 0 && mi + 1 < RB)
                    epi_store(ic<mi + 1>{}, ic<P::epi(mi, idx)>{});
                using cold = std::integral_constant<bool, FUSE>;
                if constexpr (dk == 1)
                    dma_go(A_OP{}, src_a1, ic<dj>{}, chk{}, cold{});
                else if constexpr (dk == 2)
                    dma_go(B_OP{}, src_b3, ic<dj>{}, chk{}, cold{});
                else if constexpr (dk == 3)
                    dma_go(A_OP{}, src_a2, ic<dj>{}, chk{}, cold{});
            });
        });
    };

    // ---- one K step of a partial tile (kThin) -------------------------------------------------
    // The same memory operations and barrier as a checked step, in the same order, so the waves
    // of a workgroup stay in step whichever kind of step each runs; but each row issues its
    // memory operations first (every DMA with its own M0 write and wait states) and then its 16
    // MFMAs behind one uniform branch on the wave's row mask. A skipped row block keeps stale
    // accumulators, which no store writes: its rows are past m_valid (outside the C resource) or
    // the wave's columns are all past n_valid (out-of-range chunk offsets). The row's reads fill
    // the next row's x fragments and the next step's w fragments, never the ones its MFMAs read.
    auto step_thin = [&]<int SA, int SB>(int kt) {
        kt = __builtin_amdgcn_readfirstlane(kt);
        constexpr int NX = SA ^ 1;
        constexpr int SB_NEXT = (SB + 1) % 3;
        uint32_t rows_w = __builtin_amdgcn_readfirstlane(cur.rows);
        fresh_s(rows_w); // tested next to each row's branch
        using chk = std::true_type;
        const DmaSrc src_a1 = dma_src(A_OP{}, kt + 1, chk{}); // A(kt+1)
        const DmaSrc src_b3 = dma_src(B_OP{}, kt + 3, chk{}); // B(kt+3)
        const DmaSrc src_a2 = dma_src(A_OP{}, kt + 2, chk{}); // A(kt+2)
        // DMA with its own M0 write and the SGPR wait states
        auto dma_row = [&](uint32_t dst, auto b_op, auto j, const DmaSrc &d) {
            sched_fence();
            dma16(dst + j * 4096, dma_voff(b_op, j, d, chk{}), d.rs, d.so);
            sched_fence();
        };
        sfor<0, P::rows>([&](auto mi_) {
            constexpr int mi = decltype(mi_)::value;
            sfor<0, P::slots>([&](auto idx_) {
                constexpr int idx = decltype(idx_)::value;
                constexpr int dj = P::dma_j(mi, idx);
                constexpr int dk = P::dma_kind(mi, idx) == 1 && a_dead(dj) ? 0 : P::dma_kind(mi, idx);
                if constexpr (mi == P::last && idx == P::bar) {
                    sched_fence();
                    wait_vm_lds_barrier<P::vm_at_barrier()>();
                    sched_fence();
                }
                if constexpr (P::read_a_next(mi, idx) >= 0 && mi + 1 < RB) {
                    read_frag.template operator()<A_MN, P::read_a_next(mi, idx), A_BLK>(fa[(mi + 1) & 1], a_rd[SA],
                                                                                 ic<mi + 1>{});
                    sched_fence();
                }
                if constexpr (P::read_b_next(mi, idx) >= 0) {
                    constexpr int bb = P::read_b_blk(mi, idx);
                    read_frag.template operator()<B_MN, P::read_b_next(mi, idx), B_BLK>(fb[NX][bb], b_base(SB_NEXT, ic<bb>{}),
                                                                                 ic<bb>{});
                    sched_fence();
                }
                if constexpr (P::read_a_row0(mi, idx) >= 0) {
                    read_frag.template operator()<A_MN, P::read_a_row0(mi, idx), A_BLK>(fa[0], a_rd[NX], ic<0>{});
                    sched_fence();
                }
                if constexpr (dk == 1)
                    dma_row(a_dst[NX], A_OP{}, ic<dj>{}, src_a1);
                else if constexpr (dk == 2)
                    dma_row(b_dst[SB], B_OP{}, ic<dj>{}, src_b3);
                else if constexpr (dk == 3)
                    dma_row(a_dst[SA], A_OP{}, ic<dj>{}, src_a2);
            });
            sched_fence();
            if (rows_w & (1u << mi)) {
                sfor<0, P::slots>([&](auto idx_) {
                    row_mfma.template operator()<SA, false>(mi_, idx_);
                    sched_fence();
                });
            }
            sched_fence();
        });
    };

    // ---- the persistent loop ------------------------------------------------------------------
    // Cross-tile: one prologue, before the first tile. Per-tile: a prologue at the top of every
    // tile (a single copy of it, so the fragment registers have one definition in the loop).
    if constexpr (CROSS) {
        set_stages();
        issue_prologue();
        finish_prologue.template operator()<P::lb + P::early>();
        GG_STAMP(1);
    }
    while (true) {
        if constexpr (!CROSS) {
            set_stages();
            issue_prologue();
            finish_prologue.template operator()<P::lb + P::early>();
        }
        refresh();
        const int  t_next = t + gridDim.x;
        const bool more   = t_next < total_units;
#if GG_STAMPS
        const int stamp_base = stamp_tile < 7 ? 2 + 5 * stamp_tile : kStampSlots;
        ++stamp_tile;
#endif
        GG_STAMP(stamp_base);
        // A partial tile in which this wave has at most 4 row blocks with a valid output (kThin)
        // runs its steps after the first as thin steps (step_thin) in a loop of their own; a
        // full tile never enters it. (A thin step's memory operations do not overlap its MFMAs:
        // with 5 or more rows it is no faster than a full step.) Loops in sequence, not branches
        // around whole steps, so the accumulators stay in place.
        const bool thin = kThin && __builtin_amdgcn_readfirstlane(cur.rows) <= 0xfu;
        if constexpr (CROSS) {
            // First step: stores the previous tile's accumulators while it overwrites them (to
            // nowhere for the first tile). Always the same code, so the accumulators never
            // merge across branches and stay in AGPRs.
            sfor<0, kEpiStores>([&](auto s_) { epi_store(ic<0>{}, s_); });
            step.template operator()<0, 0, true, true, true>(0);
        } else {
            step.template operator()<0, 0, true, true, false>(0);
        }
        GG_STAMP(stamp_base + 1);
        int kt = 1; // kt % 6 == 1 at the top of each block of six steps
        if constexpr (A_MN || B_MN)
            set_mn_offsets(cur);
        // Unchecked: every prefetch of the block (up to kt + 8) is a full step of this tile: before
        // T-1, which may be partial, or up to T-1 in instances without tail masks (no partial K
        // step), which thus leave 3 checked steps instead of up to 8 when T % 6 == 4.
        for (; !thin && kt + (KT ? 9 : 8) < T; kt += 6) {
            refresh();
            step.template operator()<1, 1, false, false, false>(kt);
            step.template operator()<0, 2, false, false, false>(kt + 1);
            step.template operator()<1, 0, false, false, false>(kt + 2);
            step.template operator()<0, 1, false, false, false>(kt + 3);
            step.template operator()<1, 2, false, false, false>(kt + 4);
            step.template operator()<0, 0, false, false, false>(kt + 5);
        }
        GG_STAMP(stamp_base + 2);
        cross_next = CROSS && more;
        if (cross_next)
            nxt = make_tile(t_next, tile_i + 1);
        GG_STAMP(stamp_base + 3);
        for (; !thin && kt < T; kt += 6) { // with CROSS the last three steps prefetch `nxt`
            refresh();
            step.template operator()<1, 1, false, true, false>(kt);
            if (kt + 1 < T) step.template operator()<0, 2, false, true, false>(kt + 1);
            if (kt + 2 < T) step.template operator()<1, 0, false, true, false>(kt + 2);
            if (kt + 3 < T) step.template operator()<0, 1, false, true, false>(kt + 3);
            if (kt + 4 < T) step.template operator()<1, 2, false, true, false>(kt + 4);
            if (kt + 5 < T) step.template operator()<0, 0, false, true, false>(kt + 5);
        }
        if constexpr (kThin) {
            for (; kt < T; kt += 6) {
                refresh();
                step_thin.template operator()<1, 1>(kt);
                if (kt + 1 < T) step_thin.template operator()<0, 2>(kt + 1);
                if (kt + 2 < T) step_thin.template operator()<1, 0>(kt + 2);
                if (kt + 3 < T) step_thin.template operator()<0, 1>(kt + 3);
                if (kt + 4 < T) step_thin.template operator()<1, 2>(kt + 4);
                if (kt + 5 < T) step_thin.template operator()<0, 0>(kt + 5);
            }
        }
        GG_STAMP(stamp_base + 4);
        if constexpr (CROSS) {
            if (!cross_next)
                break; // last tile of the workgroup: stored after the loop
            {
                // The next tile's first steps are in flight or in LDS, B(0) of it is in the w
                // register set T % 2 and row 0 of A(0) in fa[0]: continue without a prologue.
                prev_crs   = c_rsrc(cur);
                prev_n     = cur.n_valid;
                prev_scale = cur.scale;
                cur      = nxt;
                t        = t_next;
                ++tile_i;
                rot_a    = (rot_a + T) & 1;
                rot_b    = rot_b + T % 3;
                rot_b    = rot_b >= 3 ? rot_b - 3 : rot_b;
                set_stages();
                if (T & 1) // the first step reads w set 0
                    sfor<0, NC>([&](auto ni) { sfor<0, 2>([&](auto h) { fb[0][ni][h] = fb[1][ni][h]; }); });
                if (LAYOUT == kWgrad || TAIL) // the next group's or K range's step count
                    T = __builtin_amdgcn_readfirstlane(cur.T);
                continue;
            }
        }
        if constexpr (!CROSS) {
            // Store this tile through LDS (split-K: its partial sums to the workspace); the next
            // one starts cold at the top of the loop (the stores were issued before its DMAs and
            // complete first).
            if (splits > 1)
                store_partial(t);
            else
                epilogue_lds(cur);
            if (!more) {
                GG_STAMP_REAL(kStampRealEnd);
                GG_STAMP(kStampSlots - 1);
                return;
            }
            t   = t_next;
            ++tile_i;
            cur = make_tile(t, tile_i);
            T   = __builtin_amdgcn_readfirstlane(cur.T);
        }
    }
    if constexpr (CT) {
        // row-major accumulators: the last tile goes out from registers as well (whole 64-byte
        // pieces of rows per 4 lanes), after the trailing DMAs into LDS have landed. TAIL: a K
        // range stores its fp32 partial sums instead, as rows of a 256 x 256 slab (k * rem + tail
        // of the workspace; lane l: 32 bytes, the 8 columns of its store), with its C stores
        // dropped (no rows), and a whole tile's partial-sum stores go to a zero-length resource:
        // one branch-free exit reads the accumulators.
        GG_STAMP(kStampSlots - 2);
        wait_vm_lds_barrier<0>();
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory"); // MFMA -> VALU read distance
        Tile       tl   = cur;
        const bool part = TAIL && tl.tail >= 0;
        if constexpr (TAIL)
            tl.m_valid = part ? 0 : tl.m_valid;
        const __amdgpu_buffer_rsrc_t crs = c_rsrc(tl);
        const __amdgpu_buffer_rsrc_t prs =
            __builtin_amdgcn_make_buffer_rsrc(args.ws, static_cast<short>(0), part ? 0x7fffffff : 0, 0x00020000);
        const int poff = part ? (((tl.tail_k * rem + tl.tail) * 256 + wm * 16 + 4 * (lane >> 4)) * 256 + ecol) * 4 : 0;
        sfor<0, RB>([&](auto mi) { // short-wide tiles: 6 row blocks, and the ninth column block
            if constexpr (SWIDE)
                store_block9(mi, crs, tl.n_valid);
            sfor<0, 4>([&](auto s_) {
                if constexpr (TAIL) {
                    sfor<0, 2>([&](auto hf) {
                        asm volatile("" : "+a"(acc[mi][4 * hf]), "+a"(acc[mi][4 * hf + 1]), "+a"(acc[mi][4 * hf + 2]),
                                     "+a"(acc[mi][4 * hf + 3]));
                        const f32x4 v = {acc[mi][4 * hf][int(s_)], acc[mi][4 * hf + 1][int(s_)],
                                         acc[mi][4 * hf + 2][int(s_)], acc[mi][4 * hf + 3][int(s_)]};
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                               poff + ((32 * mi + s_) * 256) * 4 + 16 * hf, 0, 0);
                    });
                }
                store_ct(mi, s_, crs, tl.n_valid, tl.scale);
            });
        });
    } else if constexpr (CROSS) {
        GG_STAMP(kStampSlots - 2);
        epilogue_lds(cur); // TAIL: a K range's partial sums instead of its C tile
    }
    GG_STAMP_REAL(kStampRealEnd);
    GG_STAMP(kStampSlots - 1);
}

} // namespace
} // namespace gg
