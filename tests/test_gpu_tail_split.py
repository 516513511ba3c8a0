"""Tail split: the last, partial round of a cross-tile 16-bit forward plan cut into K ranges.

When a plan's tiles leave a last round of at most half the grid (config 5a: 1152 tiles on 256
workgroups, four rounds and 128 tiles), each last-round tile is computed as two K ranges by two
workgroups, which store fp32 partial sums; a second launch on the stream adds each tile's two
ranges and stores it. Checks, on NaN-prefilled outputs:
- every output within rtol = atol = 1e-2 of float32 (bench/bench_main.cpp:264-268) for K % 64 != 0
  (the second range holds the partial K step), ragged groups with an empty one, fp16, and ranges of
  one tile on different XCDs;
- the plan reports the split ("tail-split=2"; GG_TAIL_SPLIT=2 takes it wherever the plan allows
  one, GG_TAIL_SPLIT=0 turns it off), and its model takes it by itself for a shape it pays on;
- only split tiles may differ from the unsplit plan: every other output is bit-identical
  (an output's K order is the same), the split ones are within tolerance of it;
- a plan run again gives the same bits, also when two split plans alternate on one stream;
- dgrad and fp8 plans do not split.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2
GRID = 256  # MI355X CUs: one persistent workgroup per CU

# dtype, group_m, N, K, expected tail split (tiles: M-tiles x N-tiles; grid 256)
FWD = [
    (torch.bfloat16, [520] * 32, 2880, 2880, 2),   # config 5a: 1152 short tiles, 128 in the last round
    (torch.bfloat16, [4096] * 3, 1536, 2048, 2),   # 288 tiles, 32 in the last round, 32 K steps
    (torch.bfloat16, [4096], 5376, 2048, 2),       # 336 tiles, 80 in the last round
    (torch.float16, [1024] * 9, 2048, 2088, 2),    # K % 64 = 40: 33 K steps, the last range ends partial
    (torch.bfloat16, [900, 13, 2048, 0, 1500, 700, 3000], 2048, 1536, 2),  # ragged, an empty group
    (torch.bfloat16, [4096, 256], 4352, 2048, 2),  # 289 tiles: 33 in the last round, so the two
                                                   # ranges of a tile run on different XCDs
]


def _tiles(gm, n, tile_m=256):
    return sum(-(-m // tile_m) for m in gm) * -(-n // 256)


def _run_fwd(pkg, x, w, gm, monkeypatch, split):
    if split is None:
        monkeypatch.delenv("GG_TAIL_SPLIT", raising=False)
    else:
        monkeypatch.setenv("GG_TAIL_SPLIT", split)
    monkeypatch.setenv("GG_WIDE", "0")  # 256-column tiles (short-wide plans have no tail split)
    b, n, k = w.shape
    out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    be = pkg.make_mi355x_backend()
    dt = pkg.DType.BF16 if x.dtype == torch.bfloat16 else pkg.DType.FP16
    why = be.prepare(pkg.GroupedGemmProblem(dt, b, n, k, gm, x.data_ptr(), w.data_ptr(), out.data_ptr()), s)
    assert why == "", why
    return be, out, s


def _check(out, x, w, gm):
    row = 0
    for g, m in enumerate(gm):
        if m:
            ref = x[row:row + m].float() @ w[g].float().t().contiguous()
            got = out[row:row + m].float()
            assert not torch.isnan(got).any(), f"group {g}: unwritten outputs"
            bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
            assert bad == 0, f"group {g}: {bad} outputs off"
        row += m


@pytest.mark.parametrize("case", range(len(FWD)))
def test_tail_split_forward(pkg, monkeypatch, case):
    dt, gm, n, k, want_s = FWD[case]
    print(f"[tail] case {case}: dtype={dt} groups={len(gm)} N={n} K={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(300 + case)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(dt)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(dt)
    be, out, s = _run_fwd(pkg, x, w, gm, monkeypatch, "2")  # taken where the plan allows it
    detail = be.detail()
    assert f"tail-split={want_s}" in detail, detail
    be.run(s)
    torch.cuda.synchronize(DEV)
    first = out.clone()
    _check(out, x, w, gm)
    for _ in range(3):  # the counters are back at 0 after every launch
        be.run(s)
    torch.cuda.synchronize(DEV)
    assert torch.equal(first.view(torch.int16), out.view(torch.int16)), "repeated runs differ"
    be.release()
    # the unsplit plan: identical bits outside the split tiles, within tolerance inside them
    be0, out0, s0 = _run_fwd(pkg, x, w, gm, monkeypatch, "0")
    assert "tail-split" not in be0.detail(), be0.detail()
    be0.run(s0)
    torch.cuda.synchronize(DEV)
    be0.release()
    tile_rows = int(detail.split("persistent ")[1].split("x")[0])
    rem = _tiles(gm, n, tile_rows) % GRID
    differ = int((first.view(torch.int16) != out0.view(torch.int16)).sum())
    assert differ <= rem * tile_rows * 256, (differ, rem)
    f, f0 = first.float(), out0.float()
    assert bool(((f - f0).abs() <= ATOL + RTOL * f0.abs()).all())


def test_tail_split_plans_alternate(pkg, monkeypatch):
    """Two split plans alternating on one stream give their own results each time."""
    g = torch.Generator(device=DEV).manual_seed(321)
    runs = []
    for gm, n, k in (([520] * 32, 2880, 2880), ([4096] * 3, 1536, 2048)):
        x = torch.randn((sum(gm), k), generator=g, device=DEV).to(torch.bfloat16)
        w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(torch.bfloat16)
        be, out, s = _run_fwd(pkg, x, w, gm, monkeypatch, "2")
        assert "tail-split" in be.detail(), be.detail()
        be.run(s)
        torch.cuda.synchronize(DEV)
        runs.append((be, out, out.clone(), s, x, w))  # the plans read x and w: keep them alive
    for _ in range(3):
        for be, out, _, s, _, _ in runs:
            out.fill_(float("nan"))
            be.run(s)
    torch.cuda.synchronize(DEV)
    for be, out, ref, _, _, _ in runs:
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        be.release()


def test_tail_split_forced_and_off(pkg, monkeypatch):
    """GG_TAIL_SPLIT=2 takes the split wherever the plan allows it, GG_TAIL_SPLIT=1 turns it off."""
    gm, n, k = [4096] * 3, 1536, 2048
    g = torch.Generator(device=DEV).manual_seed(322)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(torch.bfloat16)
    for forced, want in (("2", "tail-split=2"), ("1", None)):
        be, out, s = _run_fwd(pkg, x, w, gm, monkeypatch, forced)
        d = be.detail()
        assert (want in d) if want else ("tail-split" not in d), d
        be.run(s)
        torch.cuda.synchronize(DEV)
        be.release()
        _check(out, x, w, gm)


def test_no_tail_split_outside_16bit_forward(pkg, monkeypatch):
    """dgrad and fp8 plans keep whole last-round tiles (the split has cross-tile 16-bit forward
    instances only)."""
    monkeypatch.delenv("GG_TAIL_SPLIT", raising=False)
    gm, n, k = [4096] * 3, 2048, 1536
    gy = torch.zeros((sum(gm), n), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((len(gm), n, k), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((sum(gm), k), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    plan = pkg.BackwardPlan("dgrad", pkg.DType.BF16, n, k, gm, gy.data_ptr(), w.data_ptr(), out.data_ptr(), s)
    assert "tail-split" not in plan.detail(), plan.detail()
    plan.release()


def test_tail_split_model(pkg, monkeypatch):
    """The plan's model splits a small last round of long tiles (32 tiles, 32 K steps) and leaves
    config 5a (128 tiles in the last round: the reduction costs more than the half tile saved)."""
    monkeypatch.delenv("GG_TAIL_SPLIT", raising=False)
    s = torch.cuda.current_stream(DEV).cuda_stream
    for gm, n, k, split in (([4096] * 3, 1536, 2048, True), ([520] * 32, 2880, 2880, False)):
        x = torch.empty((sum(gm), k), dtype=torch.bfloat16, device=DEV)
        w = torch.empty((len(gm), n, k), dtype=torch.bfloat16, device=DEV)
        out = torch.empty((sum(gm), n), dtype=torch.bfloat16, device=DEV)
        be = pkg.make_mi355x_backend()
        assert be.prepare(pkg.GroupedGemmProblem(pkg.DType.BF16, len(gm), n, k, gm, x.data_ptr(), w.data_ptr(),
                                                 out.data_ptr()), s) == ""
        assert ("tail-split=2" in be.detail()) == split, be.detail()
        be.release()
