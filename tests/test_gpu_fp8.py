"""fp8 forward grouped GEMM on the GPU (gg_prepare_fp8 through the C ABI).

bf16 out = (x[g] @ w[g]^T) * x_scale * w_scale[g] with fp8 (OCP e4m3 or e5m2) x and w and
tensor-wise scales, as the reference's vendored Primus-Turbo fp8 grouped GEMM takes them
(third_party/primus_turbo/include/primus_turbo/grouped_gemm.h:72-74, 120-123). Bar: every output
within rtol = atol = 1e-2 of the fp32 result (bench/bench_main.cpp:264-268), of the CPU oracle on
small problems and of a torch fp32 matmul of the decoded inputs on large ones; bit-exact bf16 on
small-integer inputs; NaN-prefilled outputs.
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


def _stream():
    return torch.cuda.current_stream(DEV).cuda_stream


def _fp8(shape, fmt, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(TDT[fmt])


def _run(pkg, fmt, gm, x, w, xs, ws):
    n, k = w.shape[1], w.shape[2]
    out = torch.full((x.shape[0], n), float("nan"), dtype=torch.bfloat16, device=DEV)
    xd, wd = x.to(DEV), w.to(DEV)
    xsd = torch.tensor([xs], dtype=torch.float32, device=DEV)
    wsd = torch.tensor(ws, dtype=torch.float32, device=DEV)
    plan = pkg.Fp8Plan(pkg.DType.FP8_E4M3 if fmt == 0 else pkg.DType.FP8_E5M2, n, k, gm, xd.data_ptr(),
                       wd.data_ptr(), xsd.data_ptr(), wsd.data_ptr(), out.data_ptr(), _stream())
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    return out, detail


SMALL = [
    (0, [300, 0, 17, 513], 264, 512),   # ragged and empty groups, N tail, whole K steps
    (1, [256, 256], 512, 256),          # e5m2
    (0, [1, 7, 64, 65], 8, 16),         # tiny: N = 8, K = 16 (one partial step)
    (0, [700, 300], 1000, 144),         # K % 128 = 16
    (1, [2000, 30, 900], 776, 1040),    # M tails, K % 128 = 16
]


@pytest.mark.parametrize("case", range(len(SMALL)))
def test_fp8_every_output_vs_oracle(pkg, oracle, case):
    fmt, gm, n, k = SMALL[case]
    print(f"[fp8] case {case}: fmt={fmt} group_m={gm} N={n} K={k}", flush=True)
    x = _fp8((sum(gm), k), fmt, 1)
    w = _fp8((len(gm), n, k), fmt, 2)
    ws = [0.5 + 0.25 * g for g in range(len(gm))]
    out, detail = _run(pkg, fmt, gm, x, w, 0.75, ws)
    ref = oracle.grouped_gemm_fp8(fmt, x.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), gm, 0.75, ws)
    got = out.float().cpu().numpy()
    assert not np.isnan(got).any(), f"unwritten outputs ({detail})"
    bad, mx = oracle.check(got, ref, ATOL, RTOL)
    assert bad == 0, f"{bad}/{got.size} outputs off, max abs err {mx} ({detail})"


@pytest.mark.parametrize("fmt", [0, 1])
def test_fp8_exact_small_integers(pkg, oracle, fmt):
    """fp8 inputs in {-2, ..., 2}, unit scales: every fp32 partial sum is a small integer, exact
    in bf16, so the output must match the oracle bit for bit."""
    gen = torch.Generator().manual_seed(9 + fmt)
    gm, n, k = [130, 256, 3], 264, 256
    x = torch.randint(-2, 3, (sum(gm), k), generator=gen).float().to(TDT[fmt])
    w = torch.randint(-2, 3, (len(gm), n, k), generator=gen).float().to(TDT[fmt])
    out, _ = _run(pkg, fmt, gm, x, w, 1.0, [1.0] * len(gm))
    ref = oracle.grouped_gemm_fp8(fmt, x.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), gm, 1.0,
                                  [1.0] * len(gm))
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.encode(0, ref).reshape(got.shape))


@pytest.mark.parametrize("fmt,b,m,n,k", [(0, 8, 4096, 4096, 7168), (1, 8, 4096, 7168, 2048),
                                          (0, 32, 520, 2880, 2880)])
def test_fp8_large_vs_torch_fp32(pkg, fmt, b, m, n, k):
    print(f"[fp8] large: fmt={fmt} B={b} M={m} N={n} K={k}", flush=True)
    gm = [m] * b
    x = _fp8((b * m, k), fmt, 3)
    w = _fp8((b, n, k), fmt, 4)
    ws = [1.0 / (g + 1) for g in range(b)]
    out, _ = _run(pkg, fmt, gm, x, w, 0.5, ws)
    xd, wd = x.to(DEV).float(), w.to(DEV).float()
    for g in range(b):
        ref = (xd[g * m:(g + 1) * m] @ wd[g].t().contiguous()) * (0.5 * ws[g])
        got = out[g * m:(g + 1) * m].float()
        assert not torch.isnan(got).any(), f"group {g}: unwritten outputs"
        nbad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert nbad == 0, f"group {g}: {nbad} outputs off"


@pytest.mark.parametrize("fmt", [0, 1])
def test_fp8_cross_tile_ragged(pkg, fmt):
    """More tiles than workgroups (the cross-tile variant: a tile's stores are issued in the next
    tile's first K step, scaled by the finished tile's scales) with ragged and empty groups, an N
    tail and a partial last K step; per-group scales change at every group boundary."""
    gm, n, k = [1500, 0, 77, 3000, 2513], 2056, 1040
    print(f"[fp8] cross ragged: fmt={fmt} group_m={gm} N={n} K={k}", flush=True)
    x = _fp8((sum(gm), k), fmt, 7)
    w = _fp8((len(gm), n, k), fmt, 8)
    ws = [0.25 * (g + 1) for g in range(len(gm))]
    out, detail = _run(pkg, fmt, gm, x, w, 1.5, ws)
    assert "cross-tile" in detail, detail
    xd, wd = x.to(DEV).float(), w.to(DEV).float()
    row = 0
    for g, m in enumerate(gm):
        if m:
            ref = (xd[row:row + m] @ wd[g].t().contiguous()) * (1.5 * ws[g])
            got = out[row:row + m].float()
            assert not torch.isnan(got).any(), f"group {g}: unwritten outputs"
            nbad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
            assert nbad == 0, f"group {g}: {nbad} outputs off"
        row += m


def test_fp8_torch_wrapper(pkg):
    gm = [100, 0, 412]
    x = _fp8((sum(gm), 512), 0, 5).to(DEV)
    w = _fp8((3, 264, 512), 0, 6).to(DEV)
    xs = torch.tensor([2.0], device=DEV)
    ws = torch.tensor([1.0, 1.0, 0.5], device=DEV)
    out = pkg.grouped_gemm_fp8(x, w, gm, xs, ws)
    ref = (x[100:].float() @ w[2].float().t().contiguous()) * 1.0
    assert ((out[100:].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
