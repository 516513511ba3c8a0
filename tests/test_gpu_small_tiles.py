"""Small-tile plans (128 x 128 tiles, one per workgroup, optionally split over K; gg_small.hip) for
16-bit forward problems whose 256 x 256 tiles fill at most half the GPU.

Every case runs with the small-tile plan forced (GG_SMALL=1; GG_SMALL_SPLIT sets the K ranges)
and checks every output against float32 at rtol = atol = 1e-2 (bench/bench_main.cpp:264-268),
NaN-prefilled so that an unwritten tile fails. Small-integer inputs, whose products and sums are
exact in fp32, must give the exact integer GEMM rounded to the 16-bit output, bit for bit, with
and without split-K. Shapes: ragged and empty groups, one-row groups, N with a partial 128-column
tile (N = 8, 136, 2000, 2056), K % 64 in {8, 40} and K = 8, more ranges than a K of 64 steps
divides evenly, and plans of more workgroups than CUs (a 2-step LDS ring, two workgroups per
CU).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2

# (dtype, group_m, N, K, forced K ranges or None for the plan's own)
CASES = [
    (torch.bfloat16, [512], 2880, 2880, None),
    (torch.float16, [512], 2880, 2880, None),
    (torch.bfloat16, [300, 0, 1, 129, 0, 700], 2000, 1000, None),
    (torch.bfloat16, [256, 256, 256, 256], 512, 1024, 1),
    (torch.float16, [37, 255, 128], 136, 4104, 3),
    (torch.bfloat16, [1000], 8, 8, None),
    (torch.bfloat16, [65, 200], 1024, 4136, 7),
    (torch.float16, [512, 512], 2048, 1408, None),
    (torch.bfloat16, [2048], 4096, 4096, 1),
    (torch.bfloat16, [129], 4096, 16384, 64),
    (torch.float16, [700, 0, 1300, 513], 2000, 1000, None),
    (torch.bfloat16, [300, 2000, 17], 2056, 2120, 2),
]


def _run(pkg, x, w, gm, monkeypatch, split):
    monkeypatch.setenv("GG_SMALL", "1")
    if split is None:
        monkeypatch.delenv("GG_SMALL_SPLIT", raising=False)
    else:
        monkeypatch.setenv("GG_SMALL_SPLIT", str(split))
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


@pytest.mark.parametrize("case", range(len(CASES)))
def test_small_tiles_against_fp32(pkg, monkeypatch, case):
    dt, gm, n, k, split = CASES[case]
    print(f"[small] case {case}: dtype={dt} groups={gm} N={n} K={k} split={split}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(300 + case)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(dt)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(dt)
    out, detail = _run(pkg, x, w, gm, monkeypatch, split)
    assert "small 128x128x64" in detail, detail
    tiles, steps = sum((m + 127) // 128 for m in gm) * ((n + 127) // 128), (k + 63) // 64
    if split is None:  # forced plans fill the 256 CUs with K ranges of at least 8 steps
        ranges = max(1, min(256 // tiles, steps // 8)) if tiles < 256 else 1
    else:
        ranges = -(-steps // -(-steps // min(split, steps)))
    # more workgroups than CUs: the 2-step ring, two workgroups per CU
    assert ("two-per-cu" in detail) == (tiles * ranges > 256), detail
    if split is not None:
        steps = (k + 63) // 64
        per = -(-steps // min(split, steps))
        ranges = -(-steps // per)  # no empty K range
        assert (f"split-k={ranges}" in detail) if ranges > 1 else ("split-k" not in detail), detail
    row = 0
    for gi, m in enumerate(gm):
        if m:
            ref = x[row:row + m].float() @ w[gi].float().t().contiguous()
            got = out[row:row + m].float()
            assert not torch.isnan(got).any(), f"group {gi}: unwritten outputs ({detail})"
            bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
            assert bad == 0, f"group {gi}: {bad} outputs off ({detail})"
        row += m


@pytest.mark.parametrize("split", [1, 2, 5])
def test_small_tiles_integers_exact(pkg, monkeypatch, split):
    """Inputs in {-2 .. 2}, K = 520: every partial and final sum is an integer below 2^12, exact in
    fp32, so each plan must give the exact integer GEMM rounded to the 16-bit output (RNE)."""
    gm, n, k = [100, 0, 256, 31], 392, 520
    print(f"[small] integers split={split}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(400 + split)
    xi = torch.randint(-2, 3, (sum(gm), k), generator=g, device=DEV)
    wi = torch.randint(-2, 3, (len(gm), n, k), generator=g, device=DEV)
    for dt in (torch.bfloat16, torch.float16):
        out, detail = _run(pkg, xi.to(dt), wi.to(dt), gm, monkeypatch, split)
        assert "small 128x128x64" in detail, detail
        row = 0
        for gi, m in enumerate(gm):
            if m:
                ref = (xi[row:row + m].double() @ wi[gi].double().t()).to(dt)
                assert torch.equal(out[row:row + m].view(torch.int16), ref.view(torch.int16)), (gi, detail)
            row += m


# (group_m, N, K, small tiles expected): the planner's own choice (GG_SMALL unset)
AUTO = [
    ([512], 5760, 2880, True),                # suite TestID 157: 46 tiles in 3 K ranges -> 180 small
    ([1024, 1024], 2048, 1408, True),         # TestID 112: narrow per-tile plan -> 256 small
    ([300, 300, 300], 1024, 512, True),       # pad_test 9002: 8 K steps, 72 small tiles
    ([2048], 2880, 2880, True),               # TestID 162: 368 small tiles, two per CU
    ([512], 2880, 2880, False),               # TestID 158: 92 small tiles gain too little
    ([1024], 8192, 16384, False),             # TestID 148: the persistent plan splits K
    ([4096] * 8, 4096, 7168, False),          # config 2
]


@pytest.mark.parametrize("case", range(len(AUTO)))
def test_planner_choice(pkg, monkeypatch, case):
    gm, n, k, small = AUTO[case]
    monkeypatch.delenv("GG_SMALL", raising=False)
    monkeypatch.delenv("GG_SMALL_SPLIT", raising=False)
    x = torch.zeros((sum(gm), k), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((len(gm), n, k), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((sum(gm), n), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    be = pkg.make_mi355x_backend()
    why = be.prepare(pkg.GroupedGemmProblem(pkg.DType.BF16, len(gm), n, k, gm, x.data_ptr(), w.data_ptr(),
                                            out.data_ptr()), s)
    assert why == "", why
    detail = be.detail()
    be.release()
    assert ("small 128x128x64" in detail) == small, detail
    if small:
        assert "split-k" not in detail, detail
        assert ("two-per-cu" in detail) == (sum((m + 127) // 128 for m in gm) * ((n + 127) // 128) > 256), detail
