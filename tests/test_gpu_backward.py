"""Backward grouped GEMMs on the GPU (gg_prepare_dgrad / gg_prepare_wgrad through the C ABI).

dgrad: grad_x[g] = grad_out[g] @ w[g]; wgrad: grad_w[g] = grad_out[g]^T @ x[g] (zero for an empty
group), the shapes of the reference's vendored Primus-Turbo grouped GEMM
(third_party/primus_turbo/kernels/hipblaslt_grouped_gemm.cu:80-97, 206-214). Bar: every output
within rtol = atol = 1e-2 of fp32 (bench/bench_main.cpp:264-268): of the CPU oracle on small
problems, of a torch fp32 matmul on large ones; bit-exact on small-integer inputs; NaN-prefilled
outputs, so an unwritten tile fails.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2


def _stream():
    return torch.cuda.current_stream(DEV).cuda_stream


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _rand(pkg, dt, shape, seed):
    t = torch.empty(shape, dtype=torch.bfloat16 if dt == 0 else torch.float16, device=DEV)
    pkg.fill_randn(pkg.DType(dt), t.data_ptr(), t.numel(), seed, _stream())
    return t


def _run(pkg, kind, dt, gm, n, k, go, other):
    shape = (sum(gm), k) if kind == "dgrad" else (len(gm), n, k)
    out = torch.full(shape, float("nan"), dtype=go.dtype, device=DEV)
    plan = pkg.BackwardPlan(kind, pkg.DType(dt), n, k, gm, go.data_ptr(), other.data_ptr(), out.data_ptr(),
                            _stream())
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    return out, detail


def _check(got, ref, what):
    got = got.float().cpu().numpy() if torch.is_tensor(got) else got
    assert not np.isnan(got).any(), f"{what}: unwritten outputs"
    err = np.abs(got - ref)
    bad = int((err > ATOL + RTOL * np.abs(ref)).sum())
    assert bad == 0, f"{what}: {bad}/{got.size} outputs off, max err {float(err.max())}"


SMALL = [
    (0, [300, 0, 17, 513], 264, 520),     # ragged groups, an empty one, N and K tails
    (1, [256, 256], 512, 256),            # fp16, whole tiles
    (0, [1, 7, 64, 65], 8, 8),            # tiny: N = K = 8
    (0, [700, 300], 1000, 136),           # contraction % 64 != 0 for dgrad (N = 1000)
    (0, [0, 0, 0], 64, 64),               # no rows at all: grad_w = 0, grad_x empty
    (1, [2000, 30, 900], 776, 1032),      # several tiles per workgroup
]


@pytest.mark.parametrize("case", range(len(SMALL)))
def test_dgrad_every_output_vs_oracle(pkg, oracle, case):
    dt, gm, n, k = SMALL[case]
    print(f"[backward] dgrad {case}: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    go = _rand(pkg, dt, (max(1, sum(gm)), n), 3)[:sum(gm)]
    w = _rand(pkg, dt, (len(gm), n, k), 4)
    out, detail = _run(pkg, "dgrad", dt, gm, n, k, go, w)
    if sum(gm) == 0:
        return
    ref = oracle.grouped_dgrad(dt, _bits(go), _bits(w), gm)
    _check(out, ref, f"dgrad ({detail})")


@pytest.mark.parametrize("case", range(len(SMALL)))
def test_wgrad_every_output_vs_oracle(pkg, oracle, case):
    dt, gm, n, k = SMALL[case]
    print(f"[backward] wgrad {case}: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    go = _rand(pkg, dt, (max(1, sum(gm)), n), 5)[:sum(gm)]
    x = _rand(pkg, dt, (max(1, sum(gm)), k), 6)[:sum(gm)]
    out, detail = _run(pkg, "wgrad", dt, gm, n, k, go, x)
    ref = oracle.grouped_wgrad(dt, _bits(go), _bits(x), gm)
    _check(out, ref, f"wgrad ({detail})")


@pytest.mark.parametrize("kind", ["dgrad", "wgrad"])
def test_backward_exact_small_integers(pkg, oracle, kind):
    """Inputs in {-1, 0, 1}: all fp32 partial sums are small integers, exact in the 16-bit
    output, so the GPU must match the oracle bit for bit."""
    gen = torch.Generator().manual_seed(17)
    gm, n, k = [130, 0, 256, 3], 264, 136
    go = torch.randint(-1, 2, (sum(gm), n), generator=gen).to(torch.bfloat16).to(DEV)
    other = torch.randint(-1, 2, (len(gm), n, k) if kind == "dgrad" else (sum(gm), k),
                          generator=gen).to(torch.bfloat16).to(DEV)
    out, _ = _run(pkg, kind, 0, gm, n, k, go, other)
    ref = (oracle.grouped_dgrad if kind == "dgrad" else oracle.grouped_wgrad)(0, _bits(go), _bits(other), gm)
    assert np.array_equal(_bits(out).reshape(ref.shape), oracle.encode(0, ref).reshape(ref.shape))


# MoE training shapes (the forward configs' backward passes), every output vs torch fp32.
LARGE = [
    (0, [4096] * 8, 4096, 7168),    # gate+up: grad_x [32768, 7168], grad_w [8, 4096, 7168]
    (0, [4096] * 8, 7168, 2048),    # down
    (0, [520] * 32, 2880, 2880),    # tails
    (1, [4096] * 4, 4096, 4096),
]


@pytest.mark.parametrize("case", range(len(LARGE)))
def test_backward_large_vs_torch_fp32(pkg, case):
    dt, gm, n, k = LARGE[case]
    print(f"[backward] large {case}: dtype={dt} B={len(gm)} M={gm[0]} N={n} K={k}", flush=True)
    go = _rand(pkg, dt, (sum(gm), n), 7)
    w = _rand(pkg, dt, (len(gm), n, k), 8)
    x = _rand(pkg, dt, (sum(gm), k), 9)
    gx, _ = _run(pkg, "dgrad", dt, gm, n, k, go, w)
    gw, _ = _run(pkg, "wgrad", dt, gm, n, k, go, x)
    row = 0
    for g, m in enumerate(gm):
        ref_x = go[row:row + m].float() @ w[g].float()
        ref_w = go[row:row + m].float().t().contiguous() @ x[row:row + m].float()
        for got, ref, name in ((gx[row:row + m], ref_x, "dgrad"), (gw[g], ref_w, "wgrad")):
            gotf = got.float()
            assert not torch.isnan(gotf).any(), f"{name} group {g}: unwritten"
            nbad = int(((gotf - ref).abs() > ATOL + RTOL * ref.abs()).sum())
            assert nbad == 0, f"{name} group {g}: {nbad} outputs off"
        row += m


@pytest.mark.parametrize("dt", [0, 1])
def test_wgrad_cross_tile_varying_groups(pkg, dt):
    """More tiles than workgroups with every group at least 4 K steps long: the cross-tile
    variant, whose K-step count changes at every group boundary (rows 300, 1000, 257, 700: partial
    last steps of different lengths)."""
    gm, n, k = [300, 1000, 257, 700], 2048, 2304
    print(f"[backward] wgrad cross: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    go = _rand(pkg, dt, (sum(gm), n), 5)
    x = _rand(pkg, dt, (sum(gm), k), 6)
    out, detail = _run(pkg, "wgrad", dt, gm, n, k, go, x)
    assert "cross-tile" in detail, detail
    row = 0
    for g, m in enumerate(gm):
        ref = go[row:row + m].float().t().contiguous() @ x[row:row + m].float()
        got = out[g].float()
        assert not torch.isnan(got).any(), f"group {g}: unwritten outputs ({detail})"
        nbad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert nbad == 0, f"group {g}: {nbad} outputs off ({detail})"
        row += m


@pytest.mark.parametrize("dt", [0, 1])
def test_wgrad_short_groups_cross_tile(pkg, dt):
    """Groups shorter than 4 K steps (100 and 1 rows) and an empty one next to long ones, with more
    tiles than workgroups: the cross-tile variant still runs (a short group's tiles run 4 K steps,
    the ones past its rows reading zeros), every output within tolerance and the empty group's
    gradient zero."""
    gm, n, k = [300, 100, 0, 700, 1], 4096, 2304
    print(f"[backward] wgrad short groups: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    go = _rand(pkg, dt, (sum(gm), n), 7)
    x = _rand(pkg, dt, (sum(gm), k), 8)
    out, detail = _run(pkg, "wgrad", dt, gm, n, k, go, x)
    assert "cross-tile" in detail, detail
    row = 0
    for g, m in enumerate(gm):
        ref = go[row:row + m].float().t().contiguous() @ x[row:row + m].float()
        got = out[g].float()
        assert not torch.isnan(got).any(), f"group {g}: unwritten outputs ({detail})"
        assert ((got - ref).abs() <= ATOL + RTOL * ref.abs()).all(), f"group {g} ({detail})"
        row += m


def test_torch_wrappers(pkg):
    gm, n, k = [100, 0, 412], 264, 520
    go = _rand(pkg, 1, (sum(gm), n), 1)
    w = _rand(pkg, 1, (len(gm), n, k), 2)
    x = _rand(pkg, 1, (sum(gm), k), 3)
    gx = pkg.grouped_gemm_dgrad(go, w, gm)
    gw = pkg.grouped_gemm_wgrad(go, x, gm)
    assert gx.shape == (sum(gm), k) and gw.shape == (len(gm), n, k)
    assert torch.count_nonzero(gw[1]) == 0
    ref = go[100:].float() @ w[2].float()
    assert ((gx[100:].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
