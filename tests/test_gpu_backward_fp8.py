"""fp8 backward grouped GEMMs on the GPU (gg_prepare_dgrad_fp8 / gg_prepare_wgrad_fp8, C ABI).

dgrad: grad_x[g] = (grad_out[g] @ w[g]) * grad_scale * w_scale[g]; wgrad: grad_w[g] =
(grad_out[g]^T @ x[g]) * grad_scale * x_scale[g], zero for an empty group; bf16 out. The fp8
grouped GEMMs of the reference's vendored Primus-Turbo with a transposed operand and variable K
(third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:123-130), formats e4m3 x e4m3,
e5m2 x e5m2 and the e5m2-gradient x e4m3 recipe. Bar: every output within rtol = atol = 1e-2
of the fp32 result (bench/bench_main.cpp:264-268), of the CPU oracle on small problems and of a
torch fp32 matmul of the decoded inputs on large ones; bit-exact bf16 on small-integer inputs;
NaN-prefilled outputs.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2
TDT = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}
FMTS = [(0, 0), (1, 1), (1, 0)]  # (grad_out format, other operand format), 0 e4m3, 1 e5m2


def _stream():
    return torch.cuda.current_stream(DEV).cuda_stream


def _fp8(shape, fmt, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(TDT[fmt])


def _dtype(pkg, fmt):
    return pkg.DType.FP8_E4M3 if fmt == 0 else pkg.DType.FP8_E5M2


def _run(pkg, kind, fmts, gm, n, k, go, other, gs, os_):
    shape = (sum(gm), k) if kind == "dgrad" else (len(gm), n, k)
    out = torch.full(shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    god, otd = go.to(DEV), other.to(DEV)
    gsd = torch.tensor([gs], dtype=torch.float32, device=DEV)
    osd = torch.tensor(os_, dtype=torch.float32, device=DEV)
    plan = pkg.BackwardPlan(kind, _dtype(pkg, fmts[0]), n, k, gm, god.data_ptr(), otd.data_ptr(), out.data_ptr(),
                            _stream(), other_dtype=_dtype(pkg, fmts[1]), grad_scale=gsd.data_ptr(),
                            other_scale=osd.data_ptr())
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    return out, detail


def _u8(t):
    return t.contiguous().view(torch.uint8).numpy()


def _check(oracle, got, ref, what):
    got = got.float().cpu().numpy()
    assert not np.isnan(got).any(), f"{what}: unwritten outputs"
    bad, mx = oracle.check(got, ref, ATOL, RTOL)
    assert bad == 0, f"{what}: {bad}/{got.size} outputs off, max abs err {mx}"


SMALL = [
    ([300, 0, 17, 513], 272, 528),   # ragged groups, an empty one, N tail, partial last K step
    ([256, 256], 512, 256),          # whole tiles
    ([1, 7, 64, 65], 16, 16),        # tiny: n = k = 16
    ([700, 300], 1040, 144),         # contraction % 128 = 16 for dgrad
    ([2000, 30, 900], 784, 1040),    # several tiles per workgroup
]


@pytest.mark.parametrize("fmts", FMTS)
@pytest.mark.parametrize("case", range(len(SMALL)))
def test_dgrad_fp8_every_output_vs_oracle(pkg, oracle, fmts, case):
    gm, n, k = SMALL[case]
    print(f"[fp8 backward] dgrad {case}: formats={fmts} group_m={gm} N={n} K={k}", flush=True)
    go = _fp8((sum(gm), n), fmts[0], 1)
    w = _fp8((len(gm), n, k), fmts[1], 2)
    ws = [0.5 + 0.25 * g for g in range(len(gm))]
    out, detail = _run(pkg, "dgrad", fmts, gm, n, k, go, w, 0.75, ws)
    ref = oracle.grouped_dgrad_fp8(fmts[0], fmts[1], _u8(go), _u8(w), gm, 0.75, ws)
    _check(oracle, out, ref, f"dgrad ({detail})")


@pytest.mark.parametrize("fmts", FMTS)
@pytest.mark.parametrize("case", range(len(SMALL)))
def test_wgrad_fp8_every_output_vs_oracle(pkg, oracle, fmts, case):
    gm, n, k = SMALL[case]
    print(f"[fp8 backward] wgrad {case}: formats={fmts} group_m={gm} N={n} K={k}", flush=True)
    go = _fp8((sum(gm), n), fmts[0], 3)
    x = _fp8((sum(gm), k), fmts[1], 4)
    xs = [2.0 - 0.25 * g for g in range(len(gm))]
    out, detail = _run(pkg, "wgrad", fmts, gm, n, k, go, x, 0.5, xs)
    ref = oracle.grouped_wgrad_fp8(fmts[0], fmts[1], _u8(go), _u8(x), gm, 0.5, xs)
    _check(oracle, out, ref, f"wgrad ({detail})")


@pytest.mark.parametrize("kind", ["dgrad", "wgrad"])
@pytest.mark.parametrize("fmts", FMTS)
def test_backward_fp8_exact_small_integers(pkg, oracle, kind, fmts):
    """Inputs in {-3, ..., 3} (exact in both formats), unit scales: every fp32 partial sum is an
    exact integer, so the bf16 output is the oracle's value rounded once, bit for bit."""
    gen = torch.Generator().manual_seed(17 + fmts[0] * 2 + fmts[1])
    gm, n, k = [130, 0, 256, 3], 272, 288
    go = torch.randint(-3, 4, (sum(gm), n), generator=gen).float().to(TDT[fmts[0]])
    if kind == "dgrad":
        other = torch.randint(-3, 4, (len(gm), n, k), generator=gen).float().to(TDT[fmts[1]])
        ref = oracle.grouped_dgrad_fp8(fmts[0], fmts[1], _u8(go), _u8(other), gm, 1.0, [1.0] * len(gm))
    else:
        other = torch.randint(-3, 4, (sum(gm), k), generator=gen).float().to(TDT[fmts[1]])
        ref = oracle.grouped_wgrad_fp8(fmts[0], fmts[1], _u8(go), _u8(other), gm, 1.0, [1.0] * len(gm))
    out, _ = _run(pkg, kind, fmts, gm, n, k, go, other, 1.0, [1.0] * len(gm))
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got.reshape(-1), oracle.encode(0, ref).reshape(-1))


@pytest.mark.parametrize("kind", ["dgrad", "wgrad"])
@pytest.mark.parametrize("fmts,b,m,n,k", [((1, 0), 8, 4096, 4096, 7168), ((0, 0), 8, 4096, 7168, 2048),
                                           ((1, 1), 32, 520, 2880, 2880)])
def test_backward_fp8_large_vs_torch_fp32(pkg, kind, fmts, b, m, n, k):
    """Config shapes (MoE gate+up, down, GPT-OSS tails) in forward terms: grad_out [B*M, N],
    w [B, N, K], x [B*M, K]."""
    print(f"[fp8 backward] large {kind}: formats={fmts} B={b} M={m} N={n} K={k}", flush=True)
    gm = [m] * b
    go = _fp8((b * m, n), fmts[0], 5).to(DEV)
    other = _fp8((b, n, k) if kind == "dgrad" else (b * m, k), fmts[1], 6).to(DEV)
    scales = [1.0 / (g + 1) for g in range(b)]
    out, detail = _run(pkg, kind, fmts, gm, n, k, go, other, 0.5, scales)
    gof, of = go.float(), other.float()
    for g in range(b):
        rows = slice(g * m, (g + 1) * m)
        if kind == "dgrad":
            ref = (gof[rows] @ of[g]) * (0.5 * scales[g])
            got = out[rows].float()
        else:
            ref = (gof[rows].t().contiguous() @ of[rows]) * (0.5 * scales[g])
            got = out[g].float()
        assert not torch.isnan(got).any(), f"group {g}: unwritten outputs ({detail})"
        nbad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert nbad == 0, f"group {g}: {nbad} outputs off ({detail})"


@pytest.mark.parametrize("fmts", FMTS)
def test_wgrad_fp8_cross_tile_varying_groups(pkg, fmts):
    """fp8 wgrad on the cross-tile variant: more tiles than workgroups, every group at least
    4 K steps of 128 rows, group lengths (and so K-step counts and scales) changing between
    tiles."""
    gm, n, k = [600, 1000, 513, 1400], 2048, 2304
    print(f"[fp8 backward] wgrad cross: formats={fmts} group_m={gm} N={n} K={k}", flush=True)
    go = _fp8((sum(gm), n), fmts[0], 12).to(DEV)
    x = _fp8((sum(gm), k), fmts[1], 13).to(DEV)
    xs = [0.5, 1.5, 2.0, 0.25]
    out, detail = _run(pkg, "wgrad", fmts, gm, n, k, go, x, 2.0, xs)
    assert "cross-tile" in detail, detail
    row = 0
    for g, m in enumerate(gm):
        ref = (go[row:row + m].float().t().contiguous() @ x[row:row + m].float()) * (2.0 * xs[g])
        got = out[g].float()
        assert not torch.isnan(got).any(), f"group {g}: unwritten outputs ({detail})"
        nbad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert nbad == 0, f"group {g}: {nbad} outputs off ({detail})"
        row += m


def test_dgrad_fp8_split_k(pkg, oracle, monkeypatch):
    """Few output tiles and a long contraction: split-K with the fp8 scales applied once."""
    monkeypatch.setenv("GG_SPLIT_K", "3")
    gm, n, k = [300, 0, 77], 1040, 272
    go = _fp8((sum(gm), n), 1, 7)
    w = _fp8((len(gm), n, k), 0, 8)
    ws = [0.5, 2.0, 0.25]
    out, detail = _run(pkg, "dgrad", (1, 0), gm, n, k, go, w, 1.5, ws)
    assert "split-k=3" in detail, detail
    ref = oracle.grouped_dgrad_fp8(1, 0, _u8(go), _u8(w), gm, 1.5, ws)
    _check(oracle, out, ref, detail)


def test_backward_fp8_torch_wrappers(pkg):
    gm, n, k = [100, 0, 412], 256, 512
    go = _fp8((sum(gm), n), 1, 9).to(DEV)
    w = _fp8((3, n, k), 0, 10).to(DEV)
    x = _fp8((sum(gm), k), 0, 11).to(DEV)
    gs = torch.tensor([2.0], device=DEV)
    ws = torch.tensor([1.0, 1.0, 0.5], device=DEV)
    gx = pkg.grouped_gemm_dgrad_fp8(go, w, gm, gs, ws)
    ref = (go[100:].float() @ w[2].float()) * 1.0
    assert ((gx[100:].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
    gw = pkg.grouped_gemm_wgrad_fp8(go, x, gm, gs, ws)
    assert torch.count_nonzero(gw[1].float()) == 0, "empty group's weight gradient must be zero"
    ref = (go[100:].float().t().contiguous() @ x[100:].float()) * 1.0
    assert ((gw[2].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
    with pytest.raises(pkg.GGError):  # e4m3 gradient x e5m2 weights is not a supported recipe
        pkg.grouped_gemm_dgrad_fp8(go.view(torch.uint8).view(torch.float8_e4m3fn), w.view(torch.uint8)
                                   .view(torch.float8_e5m2), gm, gs, ws)
