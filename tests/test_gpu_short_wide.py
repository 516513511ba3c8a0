"""Short-wide tiles (at most 192 x 288) for cross-tile 16-bit forward plans of short tiles.

A short plan (at most 192 rows per tile) may take tiles 288 columns wide: each wave then runs 9
column blocks instead of 8, and fewer tiles make fewer rounds (config 5a: 960 tiles of 176 x 288
instead of 1152 of 176 x 256). Every output is the same MFMA sequence over K in either tiling, so
a short-wide plan must give the bits of the 256-column short plan (GG_WIDE=0), and every output
must be within rtol = atol = 1e-2 of float32 (bench/bench_main.cpp:264-268). Outputs are
NaN-prefilled, so an unwritten output fails. GG_WIDE=1 (with GG_SHORT=1) forces the shape
wherever the plan allows it.

Cases:
- config 5a (bf16), which the plan's model picks by itself;
- fewer 5a groups in fp16, forced;
- ragged, empty and thin groups (1-112 rows, thin steps), K % 64 = 8 (the instance with tail
  masks) and N = 1000: the last N-tile is 136 columns, so the ninth column block of its wn = 0
  waves holds 8 valid columns and its wn = 1 waves none;
- N = 440: the last N-tile's wn = 1 waves hold 8 valid columns (their first block);
- N = 2000, two tiles per workgroup: the last N-tile's ninth block of the wn = 1 waves is past N,
  through the fused stores of the next tile's first step;
- fp16 with K % 64 = 8 and three tile heights' worth of groups (520, 264 and 17 rows);
- a one-round plan stays on 256-column tiles even when forced (short-wide tiles need the
  cross-tile variant).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2

# dtype, group_m, N, K, forced (GG_SHORT=1 GG_WIDE=1) or the plan's own choice, tile rows expected
CASES = [
    (torch.bfloat16, [520] * 32, 2880, 2880, False, 176),
    (torch.float16, [520] * 12, 2880, 2880, True, 176),
    (torch.bfloat16, [100, 7, 1, 64, 112, 33, 180, 0] * 12, 1000, 1096, True, 192),
    (torch.bfloat16, [300, 520, 0, 176, 1] * 20, 440, 640, True, 176),
    (torch.bfloat16, [520] * 24, 2000, 512, True, 176),
    (torch.float16, [520, 264, 17] * 30, 1152, 712, True, 176),
]


def _run(pkg, x, w, gm, wide, forced, monkeypatch):
    monkeypatch.setenv("GG_SHORT", "1" if forced else "-1")
    monkeypatch.setenv("GG_WIDE", ("1" if forced else "-1") if wide else "0")
    b, n, k = w.shape
    out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    be = pkg.make_mi355x_backend()
    dt = pkg.DType.BF16 if x.dtype == torch.bfloat16 else pkg.DType.FP16
    why = be.prepare(pkg.GroupedGemmProblem(dt, b, n, k, gm, x.data_ptr(), w.data_ptr(), out.data_ptr()), s)
    assert why == "", why
    be.run(s)
    torch.cuda.synchronize(DEV)
    detail = be.detail()
    be.release()
    return out, detail


def _check(x, w, gm, out):
    row = 0
    for gi, m in enumerate(gm):
        if m:
            ref = x[row:row + m].float() @ w[gi].float().t().contiguous()
            got = out[row:row + m].float()
            assert not torch.isnan(got).any(), f"group {gi}: unwritten outputs"
            bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
            assert bad == 0, f"group {gi}: {bad} outputs off"
        row += m


@pytest.mark.parametrize("case", range(len(CASES)))
def test_short_wide_matches_short(pkg, monkeypatch, case):
    dt, gm, n, k, forced, rows = CASES[case]
    print(f"[short-wide] case {case}: dtype={dt} groups={len(gm)} N={n} K={k} forced={forced}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(110 + case)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(dt)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(dt)
    wide, d_wide = _run(pkg, x, w, gm, True, forced, monkeypatch)
    short, d_short = _run(pkg, x, w, gm, False, forced, monkeypatch)
    assert f"persistent {rows}x288x64" in d_wide and "cross-tile" in d_wide, d_wide
    assert f"persistent {rows}x256x64" in d_short, d_short
    assert torch.equal(wide.view(torch.int16), short.view(torch.int16)), (d_wide, d_short)
    _check(x, w, gm, wide)


def test_short_wide_needs_cross_tile(pkg, monkeypatch):
    """120 short tiles (one round): per-tile variant, so 256-column tiles even with GG_WIDE=1."""
    gm, n, k = [520] * 4, 2880, 2880
    print(f"[short-wide] one round: groups={len(gm)} N={n} K={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(120)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(torch.bfloat16)
    out, detail = _run(pkg, x, w, gm, True, True, monkeypatch)
    assert "176x256x64" in detail and "per-tile" in detail, detail
    _check(x, w, gm, out)
