"""8-tile bands: plans whose every group multiplies by a B operand larger than the 256 MB Infinity
Cache (here w of 32768 x 4352 bf16, 285 MB per group) walk their tiles in bands of 8 M-tiles
instead of 4. The band changes only the order of the tiles, so each plan must give the bits of the
same plan with 4-tile bands (GG_BAND=4), and every output must be within rtol = atol = 1e-2 of
float32 (bench/bench_main.cpp:264-268). Outputs are NaN-prefilled, so an unwritten tile fails.

Cases: forward bf16 with one group of 9 M-tiles (a partial band) and with ragged and empty
groups; the same forward over device-resident group sizes; dgrad (B = w, 285 MB); fp8 e4m3
forward (w of 32768 x 8704 bytes).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2
N, K = 32768, 4352


def _band(monkeypatch, band):
    if band is None:
        monkeypatch.delenv("GG_BAND", raising=False)
    else:
        monkeypatch.setenv("GG_BAND", str(band))


def _check(got, ref, what):
    got = got.float()
    assert not torch.isnan(got).any(), f"{what}: unwritten outputs"
    bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
    assert bad == 0, f"{what}: {bad} outputs off"


@pytest.mark.parametrize("gm", [[2304], [2000, 0, 1300]], ids=["one-group", "ragged"])
def test_forward_wide_band_matches_band4(pkg, monkeypatch, gm):
    print(f"[wide band] forward groups={gm} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(120 + len(gm))
    x = torch.randn((sum(gm), K), generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn((len(gm), N, K), generator=g, device=DEV).to(torch.bfloat16)
    s = torch.cuda.current_stream(DEV).cuda_stream
    outs, details = [], []
    for band in (None, 4):
        _band(monkeypatch, band)
        out = torch.full((sum(gm), N), float("nan"), dtype=torch.bfloat16, device=DEV)
        be = pkg.make_mi355x_backend()
        why = be.prepare(pkg.GroupedGemmProblem(pkg.DType.BF16, len(gm), N, K, gm, x.data_ptr(), w.data_ptr(),
                                                out.data_ptr()), s)
        assert why == "", why
        be.run(s)
        torch.cuda.synchronize(DEV)
        details.append(be.detail())
        be.release()
        outs.append(out)
    assert "band=8" in details[0] and "band=" not in details[1], details
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), details[0]
    del outs[1]
    row = 0
    for gi, m in enumerate(gm):
        if m:
            ref = x[row:row + m].float() @ w[gi].float().t().contiguous()
            _check(outs[0][row:row + m], ref, f"group {gi}")
        row += m


def test_device_sizes_wide_band(pkg, monkeypatch):
    """Forward over device-resident group sizes: 8-tile bands from the plan's N and K alone, the
    bits of the host-size plan."""
    gm = [2000, 0, 1300]
    print(f"[wide band] device sizes groups={gm} N={N} K={K}", flush=True)
    _band(monkeypatch, None)
    g = torch.Generator(device=DEV).manual_seed(124)
    x = torch.randn((sum(gm), K), generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn((len(gm), N, K), generator=g, device=DEV).to(torch.bfloat16)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    dev = torch.full((sum(gm), N), float("nan"), dtype=torch.bfloat16, device=DEV)
    plan = pkg.DeviceLensPlan(pkg.OP_FORWARD, pkg.DType.BF16, pkg.DType.BF16, len(gm), sum(gm), N, K,
                              lens.data_ptr(), 0, x.data_ptr(), w.data_ptr(), dev.data_ptr(), s)
    plan.run(s)
    st, tiles, msg = plan.status(s)
    detail = plan.detail()
    plan.release()
    assert st == pkg.GG_OK, msg
    assert "band=8" in detail, detail
    host = torch.full_like(dev, float("nan"))
    pkg.grouped_gemm(x, w, gm, out=host)
    torch.cuda.synchronize(DEV)
    assert torch.equal(dev.view(torch.int16), host.view(torch.int16)), detail


def test_dgrad_wide_band_matches_band4(pkg, monkeypatch):
    gm = [2304, 0, 700]
    n, k = N, K  # forward terms: grad_out [M, 32768], w [B, 32768, 4352], grad_x [M, 4352]
    print(f"[wide band] dgrad groups={gm} N={n} K={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(125)
    go = torch.randn((sum(gm), n), generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(torch.bfloat16)
    s = torch.cuda.current_stream(DEV).cuda_stream
    outs, details = [], []
    for band in (None, 4):
        _band(monkeypatch, band)
        out = torch.full((sum(gm), k), float("nan"), dtype=torch.bfloat16, device=DEV)
        plan = pkg.BackwardPlan("dgrad", pkg.DType.BF16, n, k, gm, go.data_ptr(), w.data_ptr(), out.data_ptr(), s)
        plan.run(s)
        torch.cuda.synchronize(DEV)
        details.append(plan.detail())
        plan.release()
        outs.append(out)
    assert "band=8" in details[0] and "band=" not in details[1], details
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), details[0]
    row = 0
    for gi, m in enumerate(gm):
        if m:
            _check(outs[0][row:row + m], go[row:row + m].float() @ w[gi].float(), f"group {gi}")
        row += m


def test_fp8_wide_band_matches_band4(pkg, monkeypatch):
    gm, k = [2304], 8704  # w of 32768 x 8704 e4m3 bytes: 285 MB
    print(f"[wide band] fp8 groups={gm} N={N} K={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(126)
    x = (torch.randn((sum(gm), k), generator=g, device=DEV) * 0.5).to(torch.float8_e4m3fn)
    w = (torch.randn((len(gm), N, k), generator=g, device=DEV) * 0.5).to(torch.float8_e4m3fn)
    xs = torch.tensor([0.5], device=DEV)
    ws = torch.tensor([1.5], device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    outs, details = [], []
    for band in (None, 4):
        _band(monkeypatch, band)
        out = torch.full((sum(gm), N), float("nan"), dtype=torch.bfloat16, device=DEV)
        plan = pkg.Fp8Plan(pkg.DType.FP8_E4M3, N, k, gm, x.data_ptr(), w.data_ptr(), xs.data_ptr(), ws.data_ptr(),
                           out.data_ptr(), s)
        plan.run(s)
        torch.cuda.synchronize(DEV)
        details.append(plan.detail())
        plan.release()
        outs.append(out)
    assert "band=8" in details[0] and "band=" not in details[1], details
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), details[0]
    del outs[1]
    ref = (x.float() @ w[0].float().t().contiguous()) * (xs[0] * ws[0])
    _check(outs[0], ref, "group 0")
