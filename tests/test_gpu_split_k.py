"""Split-K on the GPU: problems with few output tiles and long K, through the C ABI.

Each tile's K steps are cut into S ranges computed by different workgroups; the fp32 partial
sums are added in split order by a second kernel, then scaled (fp8) and converted. hipBLASLt's
stream-K kernels win such shapes in the reference's sweep (README.md:56-58); the reference's
ck_tile backend has no split (ck_grouped_gemm.cpp:166-188 sets k_batch = 1). Bar: every output
within rtol = atol = 1e-2 of the CPU oracle's fp32 result (bench/bench_main.cpp:264-268) on
NaN-prefilled outputs (an unwritten tile fails), the same bits on repeated runs, bit-exact
outputs on small-integer inputs, and agreement with the unsplit kernel to the same tolerance.
GG_SPLIT_K forces the split count (the library reads it at prepare).
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


def _forward(pkg, dt, gm, x, w, runs=1):
    n, k = w.shape[1], w.shape[2]
    out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device=DEV)
    be = pkg.make_mi355x_backend()
    prob = pkg.GroupedGemmProblem(pkg.DType(dt), len(gm), n, k, list(gm), x.data_ptr(), w.data_ptr(),
                                  out.data_ptr())
    why = be.prepare(prob, _stream())
    assert why == "", why
    outs = []
    for _ in range(runs):
        be.run(_stream())
        torch.cuda.synchronize(DEV)
        outs.append(out.clone())
    detail = be.detail()
    be.release()
    return outs if runs > 1 else outs[0], detail


def _check(oracle, got, ref, what):
    got = got.float().cpu().numpy() if torch.is_tensor(got) else got
    assert not np.isnan(got).any(), f"{what}: unwritten outputs"
    bad, mx = oracle.check(got, ref, ATOL, RTOL)
    assert bad == 0, f"{what}: {bad}/{got.size} outputs off, max abs err {mx}"


# (dtype, group_m, N, K, forced splits)
FORCED = [
    (0, [256], 256, 1024, 2),            # one tile, two ranges of 8 K steps
    (0, [200, 0, 57], 264, 1000, 3),     # M and N tails, an empty group, partial last K step
    (1, [300], 520, 2880, 7),            # fp16, 45 K steps in 7 uneven ranges
    (0, [1, 7], 8, 72, 2),               # 2 K steps, the second partial (8 values)
    (0, [513, 64], 776, 4104, 16),       # 65 K steps, the last one 8 values long
    (1, [129], 136, 264, 5),             # 5 K steps, one per range, partial last
    (0, [2048] * 4, 1024, 512, 8),       # 128 tiles x 8 ranges: several units per workgroup
    (0, [300, 40], 512, 512, 64),        # asked for more ranges than K steps: one step each
    # 48 tiles x 8 ranges = 384 units on 256 workgroups: a workgroup's second unit wraps to an
    # earlier tile of an earlier group (the kernel's group scan has to restart)
    (0, [512, 512], 2880, 1024, 8),
]


@pytest.mark.parametrize("case", range(len(FORCED)))
def test_forced_split_every_output_vs_oracle(pkg, oracle, monkeypatch, case):
    dt, gm, n, k, sp = FORCED[case]
    print(f"[split-k] forward case {case}: dtype={dt} group_m={gm} N={n} K={k} splits={sp}", flush=True)
    monkeypatch.setenv("GG_SPLIT_K", str(sp))
    x = _rand(pkg, dt, (sum(gm), k), 1)
    w = _rand(pkg, dt, (len(gm), n, k), 2)
    out, detail = _forward(pkg, dt, gm, x, w)
    want = min(sp, -(-k // 64))
    assert f"split-k={want}" in detail, detail
    ref = oracle.grouped_gemm(dt, _bits(x), _bits(w), gm)
    _check(oracle, out, ref, detail)


def test_split_matches_unsplit(pkg, monkeypatch):
    """The same problem with and without split-K: both within tolerance of each other (they
    differ only in the fp32 summation order)."""
    gm, n, k = [384, 128], 768, 2304
    x = _rand(pkg, 0, (sum(gm), k), 5)
    w = _rand(pkg, 0, (len(gm), n, k), 6)
    monkeypatch.setenv("GG_SPLIT_K", "1")
    one, d1 = _forward(pkg, 0, gm, x, w)
    assert "split-k" not in d1, d1
    monkeypatch.setenv("GG_SPLIT_K", "6")
    six, d6 = _forward(pkg, 0, gm, x, w)
    assert "split-k=6" in d6, d6
    a, b = one.float(), six.float()
    assert ((a - b).abs() <= ATOL + RTOL * a.abs()).all()


@pytest.mark.parametrize("dt", [0, 1])
def test_split_exact_small_integers(pkg, oracle, monkeypatch, dt):
    """Small-integer inputs: every partial sum is an exact integer in fp32, so the split sum is
    the exact product, bit for bit in the 16-bit output."""
    monkeypatch.setenv("GG_SPLIT_K", "4")
    gen = torch.Generator().manual_seed(11 + dt)
    td = torch.bfloat16 if dt == 0 else torch.float16
    gm, n, k = [130, 256, 3], 264, 520
    x = torch.randint(-2, 3, (sum(gm), k), generator=gen).to(td).to(DEV)
    w = torch.randint(-2, 3, (len(gm), n, k), generator=gen).to(td).to(DEV)
    out, detail = _forward(pkg, dt, gm, x, w)
    assert "split-k=4" in detail, detail
    ref = oracle.grouped_gemm(dt, _bits(x), _bits(w), gm)
    assert np.array_equal(_bits(out), oracle.encode(dt, ref).reshape(out.shape))


def test_auto_split_low_occupancy_shape(pkg, oracle):
    """The suite's weakest shape (shapes/full.csv TestID 158: one group, 512 x 2880 x 2880,
    24 tiles for 256 CUs) takes split-K by itself; repeated runs give the same bits (the
    partial sums are added in a fixed order)."""
    gm, n, k = [512], 2880, 2880
    x = _rand(pkg, 0, (512, k), 1)
    w = _rand(pkg, 0, (1, n, k), 2)
    outs, detail = _forward(pkg, 0, gm, x, w, runs=3)
    assert "split-k=" in detail, detail
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16)), "runs differ"
    s = oracle.make_samples(1, n, gm, 256)
    ref = oracle.sampled(0, _bits(x), _bits(w), s)
    got = outs[0][torch.from_numpy(s[:, 0]).to(DEV), torch.from_numpy(s[:, 1]).to(DEV)].float().cpu().numpy()
    _check(oracle, got, ref, detail)
    full = (x.float() @ w[0].float().t().contiguous())
    assert ((outs[0].float() - full).abs() <= ATOL + RTOL * full.abs()).all()


@pytest.mark.parametrize("sp", [None, 3])
def test_dgrad_split(pkg, oracle, monkeypatch, sp):
    """dgrad with few output tiles: grad_x [sum(M), K] = grad_out [sum(M), N] @ w[g] [N, K],
    contraction N split (auto, or forced to 3 ranges with a partial last step)."""
    if sp is not None:
        monkeypatch.setenv("GG_SPLIT_K", str(sp))
    gm, n, k = [300, 0, 200], 2056, 520
    go = _rand(pkg, 0, (sum(gm), n), 3)
    w = _rand(pkg, 0, (len(gm), n, k), 4)
    out = torch.full((sum(gm), k), float("nan"), dtype=torch.bfloat16, device=DEV)
    plan = pkg.BackwardPlan("dgrad", pkg.DType.BF16, n, k, gm, go.data_ptr(), w.data_ptr(), out.data_ptr(),
                            _stream())
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    assert "split-k=" in detail, detail
    ref = oracle.grouped_dgrad(0, _bits(go), _bits(w), gm)
    _check(oracle, out, ref, detail)


@pytest.mark.parametrize("fmt,sp", [(0, 4), (1, 3)])
def test_fp8_split(pkg, oracle, monkeypatch, fmt, sp):
    """fp8 forward with split-K: the per-group scales are applied once, to the summed partials."""
    monkeypatch.setenv("GG_SPLIT_K", str(sp))
    tdt = torch.float8_e4m3fn if fmt == 0 else torch.float8_e5m2
    gen = torch.Generator().manual_seed(21 + fmt)
    gm, n, k = [300, 0, 77], 264, 1040
    x = torch.randn((sum(gm), k), generator=gen).to(tdt)
    w = torch.randn((len(gm), n, k), generator=gen).to(tdt)
    ws = [0.5, 2.0, 0.25]
    out = torch.full((sum(gm), n), float("nan"), dtype=torch.bfloat16, device=DEV)
    xd, wd = x.to(DEV), w.to(DEV)
    xs = torch.tensor([1.5], dtype=torch.float32, device=DEV)
    wsd = torch.tensor(ws, dtype=torch.float32, device=DEV)
    plan = pkg.Fp8Plan(pkg.DType.FP8_E4M3 if fmt == 0 else pkg.DType.FP8_E5M2, n, k, gm, xd.data_ptr(),
                       wd.data_ptr(), xs.data_ptr(), wsd.data_ptr(), out.data_ptr(), _stream())
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    assert f"split-k={sp}" in detail, detail
    ref = oracle.grouped_gemm_fp8(fmt, x.view(torch.uint8).numpy(), w.view(torch.uint8).numpy(), gm, 1.5, ws)
    _check(oracle, out, ref, detail)
