"""The transposed (MN-major) operand layouts of the kernel and the row-major accumulators' B
layout and stores, checked on the CPU.

csrc/gg_kernel_impl.h stages an MN-major operand's K step in LDS with LDS DMAs (64 lanes x 16
bytes at M0 + 16 * lane) and reads fragments back with transposed LDS reads. This test restates
the kernel's lane formulas (dma_off / mn_col, the fragment bases mn / mn_half and read_frag's
offsets), simulates the DMAs into a 32 KB stage and the reads out of it, and checks:
- every byte of the stage is written exactly once, from the step's rows and the tile's columns;
- every lane's fragment holds, for MN element i of its column block, the contraction values of
  the K-major fragment's order (fp8: lane group q takes 16-byte chunks 2q + (kh ^ (q & 1)),
  16-bit: chunk 4 kh + q), so both operands of an MFMA see the same K order;
- fp8: every 4 consecutive lanes of a DMA read one 64-byte run of one stored row (the DMA unit's
  cost is one cycle per 4-lane group and cache line, as a DMA microbenchmark measured);
- no bank holds more than 2 of a read's 4-byte words (64 banks; 512 bytes per read).
The transposed reads follow the lane mapping pinned on the GPU: ds_read_b64_tr_b8 gives byte j of
lane i from byte i%8 of source lane 2j + i/8 of its 16-lane group, ds_read_b64_tr_b16 element j of
lane i from element i%4 of source lane 4j + i/4. The GPU parity tests run the kernel itself.
Row-major accumulators (GG_CT): B's DMAs fill each LDS byte once, every gathered fragment read
finds its stored row and chunk, a ds_read_b128 pass (two 8-lane groups whose lane / 16 differ in
bit 0) hits 64 distinct banks (and would hit 32 twice without the row swap, as the counters
measured), every output of a tile is stored once from the accumulator holding it, and the
partial-sum slabs are row-major as the tail reduction reads them.
"""
import collections
import itertools

import pytest


# ---- fp8 MN-major (K step: 128 stored rows x 256 columns of one byte) ----------------------------
def f8_dma(wave, j, lane):
    """(stored row, column) read by lane `lane` of DMA j of wave `wave` (dma_off, mn_col)."""
    sw = (j >> 1) & 1
    rlo = (4 * wave + (lane >> 4)) & 7
    col = (8 * (((lane & 15) >> 3) ^ sw) + ((lane & 7) ^ rlo)) * 16
    row = 16 * (j ^ sw) + 4 * wave + (lane >> 4)
    return row, col


def f8_read(h, lane, blk, kh, half):
    """LDS byte address of source lane `lane` in read (kh, half) of column block 8 h + blk."""
    q, s = lane >> 4, lane & 15
    base = q * 8192 + (s >> 1) * (256 + 16) + (s & 1) * 8 + 128 * (h ^ (q & 1))
    return (base ^ (16 * blk)) + kh * 4096 + half * 2048


# ---- 16-bit MN-major (K step: 64 stored rows x 256 columns of two bytes) ------------------------
def h_dma(wave, j, lane):
    mn_c = (wave & 1) * 8 + (lane >> 3)
    col = (mn_c ^ (j & 1)) * 16 + (lane & 1) * 8  # elements
    row = 4 * (2 * j + (wave >> 1)) + ((lane & 7) >> 1)
    return row, col


def h_read(h, lane, blk, kh, half):
    q = lane >> 4
    base = [h * 1024 + q * 4096 + (lane & 15) * 8 + (-128 if k_ else 128) * (q & 1) for k_ in (0, 1)]
    return base[blk & 1] + kh * 16384 + half * 2048 + blk * 128


def stage(dma, elem_bytes):
    """LDS byte -> (stored row, column element) after the 32 DMAs (4 waves x 8) of one K step."""
    lds = {}
    for w, j in itertools.product(range(4), range(8)):
        for lane in range(64):
            row, col = dma(w, j, lane)
            assert 0 <= col < 256
            a = 4096 * j + 1024 * w + 16 * lane
            for b in range(16):
                assert a + b not in lds, "LDS byte written twice"
                lds[a + b] = (row, col + b // elem_bytes)
    assert sorted(lds) == list(range(32768))
    return lds


def banks_worst(addrs):
    cnt = collections.Counter()
    for a in addrs:
        for d in range(2):
            cnt[((a // 4) + d) % 64] += 1
    return max(cnt.values())


def check_fp8_reads(lds):
    for h, blk, kh, half in itertools.product(range(2), range(8), range(2), range(2)):
        addrs = [f8_read(h, lane, blk, kh, half) for lane in range(64)]
        assert all(a % 8 == 0 and 0 <= a <= 32768 - 8 for a in addrs)
        assert banks_worst(addrs) <= 2
        for lane in range(64):
            q, i = lane >> 4, lane & 15
            chunk = 2 * q + (kh ^ (q & 1))  # the K-major fp8 fragment's chunk for this k-half
            for t in range(8):
                src = addrs[16 * q + 2 * t + i // 8]
                row, col = lds[src + i % 8]
                assert (row, col) == (16 * chunk + 8 * half + t, 16 * (8 * h + blk) + i)


def test_fp8_mn_major_layout():
    lds = stage(f8_dma, 1)
    assert sorted({v[0] for v in lds.values()}) == list(range(128))
    check_fp8_reads(lds)


def test_fp8_mn_major_dma_reads_64_byte_runs():
    for w, j in itertools.product(range(4), range(8)):
        for g in range(16):
            cells = [f8_dma(w, j, 4 * g + x) for x in range(4)]
            rows = {r for r, _ in cells}
            cols = sorted(c for _, c in cells)
            assert len(rows) == 1 and cols[0] % 64 == 0 and cols == [cols[0] + 16 * x for x in range(4)]


def test_16bit_mn_major_layout():
    lds = stage(h_dma, 2)
    assert sorted({v[0] for v in lds.values()}) == list(range(64))
    for h, blk, kh, half in itertools.product(range(2), range(8), range(2), range(2)):
        addrs = [h_read(h, lane, blk, kh, half) for lane in range(64)]
        assert all(a % 8 == 0 and 0 <= a <= 32768 - 8 for a in addrs)
        assert banks_worst(addrs) <= 2
        for lane in range(64):
            q, i = lane >> 4, lane & 15
            for t in range(4):
                src = addrs[16 * q + 4 * t + i // 4]
                row, col = lds[src + 2 * (i % 4)]
                # chunk 4 kh + q of 8 contraction values, half of it per read
                assert (row, col) == (8 * (4 * kh + q) + 4 * half + t, 16 * (8 * h + blk) + i)


def _planted_f8_dma(wave, j, lane):
    row, col = f8_dma(wave, j, lane)
    return row, col ^ 16 if lane == 5 else col  # one lane reads the neighbouring column block


def test_layout_check_catches_a_planted_mistake():
    with pytest.raises(AssertionError):
        check_fp8_reads(stage(_planted_f8_dma, 1))


# ---- row-major accumulators (whole-tile 16-bit forward, GG_CT) ----------------------------------
# B (w) stage: 256 stored rows (tile columns) x 128 bytes of one K step. LDS row p holds stored
# row p ^ ((p >> 3) & 1) and keeps its chunk c at slot c ^ ((p >> 3) & 7) (dma_off with ct,
# frag_b / frag_bo in csrc/gg_kernel_impl.h). A fragment of column block ni (a wave's column half
# wn) gathers stored rows wn * 128 + 8 (l % 16) + ni, chunk 4 kh + l / 16.
def ct_dma(wave, j, lane, swap=True):
    """(stored row, logical chunk) of lane `lane` of B's DMA j of wave `wave`."""
    r = (lane >> 3) ^ ((wave & 1) if swap else 0)
    return (4 * j + wave) * 8 + r, (lane & 7) ^ ((4 * j + wave) & 7)


def ct_read(wn, ni, kh, lane, swap=True):
    """LDS byte address of lane `lane`'s read (k-half kh) of column block ni (frag_b / frag_bo)."""
    fr_row, q = lane & 15, lane >> 4
    odd = (fr_row & 1) if swap else 0
    ct_off = (8 * fr_row + odd) * 128 + (((kh * 4 + q) ^ (fr_row & 7)) * 16)
    base_even = wn * 128 * 128 + ct_off
    base_odd = base_even - odd * 256
    return (base_odd if ni & 1 else base_even) + ni * 128


def ct_stage(swap=True):
    lds = {}
    for w, j in itertools.product(range(4), range(8)):
        for lane in range(64):
            row, chunk = ct_dma(w, j, lane, swap)
            a = 4096 * j + 1024 * w + 16 * lane
            assert a not in lds
            lds[a] = (row, chunk)
    assert sorted(lds) == list(range(0, 32768, 16))
    assert sorted(lds.values()) == [(r, c) for r in range(256) for c in range(8)]
    return lds


def read_pass_worst(addrs):
    """Worst bank load of a ds_read_b128, served in passes of two 8-lane groups whose lane / 16
    differ in bit 0 (lanes 0-7 with 16-23, 8-15 with 24-31, ...): 16 lanes x 4 banks of 64."""
    worst = 0
    for g0 in (0, 8, 32, 40):
        cnt = collections.Counter()
        for lane in list(range(g0, g0 + 8)) + list(range(g0 + 16, g0 + 24)):
            for d in range(4):
                cnt[((addrs[lane] // 4) + d) % 64] += 1
        worst = max(worst, max(cnt.values()))
    return worst


def check_ct_reads(lds, swap=True):
    worst = 0
    for wn, ni, kh in itertools.product(range(2), range(8), range(2)):
        addrs = [ct_read(wn, ni, kh, lane, swap) for lane in range(64)]
        for lane, a in enumerate(addrs):
            assert a % 16 == 0 and 0 <= a < 32768
            assert lds[a] == (wn * 128 + 8 * (lane & 15) + ni, kh * 4 + (lane >> 4))
        worst = max(worst, read_pass_worst(addrs))
    return worst


def test_row_major_acc_b_layout_conflict_free():
    lds = ct_stage()
    assert check_ct_reads(lds) == 1


def test_row_major_acc_b_layout_without_the_row_swap_conflicts():
    """The layout before the row swap: the same words, but every read pass puts its 16 requests on
    one half of the banks (2-way; measured 33 % SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE)."""
    assert check_ct_reads(ct_stage(swap=False), swap=False) == 2


def test_read_pass_model_on_the_k_major_layout():
    """The K-major fragment reads of A (and of B in C^T instances), chunk c at c ^ (r % 8), rows
    16 ni + l % 16: conflict-free under the same pass model (measured 0.0-0.2 %)."""
    for ni, kh in itertools.product(range(8), range(2)):
        addrs = [(16 * ni + (lane & 15)) * 128 + (((4 * kh + (lane >> 4)) ^ (lane & 7)) * 16) for lane in range(64)]
        assert read_pass_worst(addrs) == 1


def test_row_major_acc_b_dma_k_tail_chunks():
    """The partial last K step masks B's DMA lanes by the logical chunk of their DMA's parity
    (ktail_ct[j & 1]): (l % 8) ^ ((4 p + wave) % 8) for p = j % 2."""
    for w, j, lane in itertools.product(range(4), range(8), range(64)):
        _, chunk = ct_dma(w, j, lane)
        p = j & 1
        assert chunk == (lane & 7) ^ ((4 * p + w) & 7)


def test_row_major_acc_stores_cover_the_tile():
    """store_ct: store s of row block mi, lane l writes row 16 (2 mi + wm) + 4 (l / 16) + s at
    columns wn * 128 + 8 (l % 16) .. +7, element s of column blocks 0..7 (column slot l % 16 of
    block ni = column 8 (l % 16) + ni); the MFMA output lane l of block (mi, ni) holds rows
    4 (l / 16) + e, column slot l % 16. Every output of the 256 x 256 tile is written once, from
    the accumulator that holds it, and 4 consecutive lanes write 64 contiguous bytes of a row."""
    seen = {}
    for wave, mi, s, lane in itertools.product(range(4), range(8), range(4), range(64)):
        wm, wn, q = wave >> 1, wave & 1, lane >> 4
        row = (wm * 16 + 4 * q) + 32 * mi + s
        col0 = wn * 128 + 8 * (lane & 15)
        for ni in range(8):
            # the accumulator element (wave, mi, ni, lane, e = s): D[4 q + e][l % 16] of block (mi, ni)
            out = (16 * (2 * mi + wm) + 4 * q + s, wn * 128 + 8 * (lane & 15) + ni)
            assert out == (row, col0 + ni)
            assert out not in seen
            seen[out] = (wave, mi, ni, lane, s)
    assert len(seen) == 256 * 256
    for lane0 in range(0, 64, 4):
        cols = [8 * ((lane0 + x) & 15) for x in range(4)]
        rows = {(lane0 + x) >> 4 for x in range(4)}
        assert len(rows) == 1 and cols == [cols[0] + 8 * x for x in range(4)] and cols[0] % 32 == 0


def test_row_major_acc_partial_slab_order():
    """Tail-split K ranges store fp32 partial sums as a row-major 256 x 256 slab (float index
    row * 256 + column); tail_reduce_kernel's position p reads floats 4 p .. 4 p + 3 as row p / 64,
    columns 4 (p % 64) .. +3."""
    written = set()
    for wave, mi, s, lane, hf in itertools.product(range(4), range(8), range(4), range(64), range(2)):
        wm, wn, q = wave >> 1, wave & 1, lane >> 4
        ecol = wn * 128 + 8 * (lane & 15)
        byte = (((wm * 16 + 4 * q) * 256 + ecol) * 4) + ((32 * mi + s) * 256) * 4 + 16 * hf
        for t in range(4):
            f = byte // 4 + t
            ni = 4 * hf + t
            assert f == (16 * (2 * mi + wm) + 4 * q + s) * 256 + ecol + ni
            written.add(f)
    assert written == set(range(65536))
    for p in range(16384):
        assert 4 * p == (p >> 6) * 256 + 4 * (p & 63)
