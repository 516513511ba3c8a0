"""Short tiles (at most 192 x 256) for forward problems whose groups keep their M-tile counts.

When every group keeps its number of M-tiles with fewer rows per tile (a multiple of 16, at most
192), the plan may take tiles of that many rows: config 5a's groups of 520 rows become three
tiles of 176 rows instead of 256 + 256 + 8. Each wave then runs its first 6 interleaved row
blocks. Every output is the same MFMA sequence over K in either tiling, so a short plan must
give the bits of the 256-row plan (GG_SHORT=0), and every output must be within rtol = atol =
1e-2 of float32 (bench/bench_main.cpp:264-268). Outputs are NaN-prefilled. GG_SHORT=1 forces
short tiles wherever the tile counts allow.

Cases:
- config 5a (cross-tile), which the plan's model picks by itself;
- ragged and empty groups with a one-round per-tile plan and K % 64 = 8, in fp16;
- enough tiles for the cross-tile variant, with thin short tiles (groups of 1-112 rows) and a
  column tail;
- 513-row groups next to 1-row ones (160 tiles: one round, not split);
- dgrad on config 5a's shapes (bf16, fp16), whose output rows are the tokens.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2

# dtype, group_m, N, K, forced (GG_SHORT=1) or the plan's own choice, tile rows expected
CASES = [
    (torch.bfloat16, [520] * 32, 2880, 2880, False, 176),
    (torch.float16, [300, 0, 260, 130], 1000, 200, True, 160),
    (torch.bfloat16, [100, 7, 1, 64, 112, 33] * 12, 1160, 448, True, 112),
    (torch.bfloat16, [513, 1] * 20, 512, 1088, True, 176),
]


def _run(pkg, x, w, gm, env, monkeypatch):
    if env is None:
        monkeypatch.delenv("GG_SHORT", raising=False)
    else:
        monkeypatch.setenv("GG_SHORT", env)
    # bit-identity needs the same K order per output in both plans: no tail split (it sums the
    # K ranges of other last-round tiles in the two tilings); 256-column tiles (short-wide tiles
    # are tests/test_gpu_short_wide.py's)
    monkeypatch.setenv("GG_TAIL_SPLIT", "0")
    monkeypatch.setenv("GG_WIDE", "0")
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
def test_short_tiles_match_wide(pkg, monkeypatch, case):
    dt, gm, n, k, forced, rows = CASES[case]
    print(f"[short] case {case}: dtype={dt} groups={len(gm)} N={n} K={k} forced={forced}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(70 + case)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(dt)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(dt)
    short, d_short = _run(pkg, x, w, gm, "1" if forced else None, monkeypatch)
    wide, d_wide = _run(pkg, x, w, gm, "0", monkeypatch)
    assert f"persistent {rows}x256x64" in d_short, d_short
    assert "persistent 256x" in d_wide, d_wide
    assert torch.equal(short.view(torch.int16), wide.view(torch.int16)), (d_short, d_wide)
    row = 0
    for gi, m in enumerate(gm):
        ref = x[row:row + m].float() @ w[gi].float().t().contiguous()
        got = short[row:row + m].float()
        assert not torch.isnan(got).any(), f"group {gi}: unwritten outputs"
        bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert bad == 0, f"group {gi}: {bad} outputs off"
        row += m


def _env(monkeypatch, env):
    if env is None:
        monkeypatch.delenv("GG_SHORT", raising=False)
    else:
        monkeypatch.setenv("GG_SHORT", env)


def _dgrad(pkg, go, w, gm, env, monkeypatch):
    # grad_x [sum(M), K] = grad_out [sum(M), N] @ w[g] [N, K]: output rows are the group's tokens
    _env(monkeypatch, env)
    b, n, k = w.shape
    out = torch.full((go.shape[0], k), float("nan"), dtype=go.dtype, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    dt = pkg.DType.BF16 if go.dtype == torch.bfloat16 else pkg.DType.FP16
    plan = pkg.BackwardPlan("dgrad", dt, n, k, gm, go.data_ptr(), w.data_ptr(), out.data_ptr(), s)
    plan.run(s)
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    return out, detail


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_short_tiles_dgrad(pkg, monkeypatch, dt):
    gm, n, k = [520] * 32, 2880, 2880  # config 5a's shapes: the model picks short tiles
    print(f"[short] dgrad: dtype={dt} groups={len(gm)} N={n} K={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(80)
    go = torch.randn((sum(gm), n), generator=g, device=DEV).to(dt)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(dt)
    short, d_short = _dgrad(pkg, go, w, gm, None, monkeypatch)
    wide, d_wide = _dgrad(pkg, go, w, gm, "0", monkeypatch)
    assert "persistent 176x256x64" in d_short, d_short
    assert "persistent 256x256x64" in d_wide, d_wide
    assert torch.equal(short.view(torch.int16), wide.view(torch.int16)), (d_short, d_wide)
    row = 0
    for gi, m in enumerate(gm):
        ref = go[row:row + m].float() @ w[gi].float()
        got = short[row:row + m].float()
        assert not torch.isnan(got).any(), f"group {gi}: unwritten outputs"
        bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert bad == 0, f"group {gi}: {bad} outputs off"
        row += m

