"""The transposed (MN-major) operand layouts of the kernel, checked on the CPU.

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
