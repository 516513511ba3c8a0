"""Seeded random shapes through every pass, against a torch fp32 reference of the same op.

Each case draws B groups of ragged sizes (some empty), N and K multiples of 8 up to 3200, bf16 or
fp16, and one of the forward, dgrad and wgrad passes, with the group sizes on the host or on the
device. The planner picks whatever it picks for the shape (cross-tile or per-tile, split-K, tail
split, short, short-wide, narrow or small tiles, descriptors or the table walk, masks or none), so the
sweep covers the plan boundaries that hand-picked shapes may miss. Every output is checked at
|got - ref| <= 1e-2 + 1e-2 * |ref| (bench/bench_main.cpp:264-268); the host-size forward
output is NaN-prefilled, so an unwritten tile fails.

fp8 cases: the library's recipes (e4m3 and e5m2 forward, e5m2-gradient x e4m3 and matching
formats for dgrad and wgrad; N and K multiples of 16) with random tensor-wise scales, against the fp32 product of the
decoded operands times the scales.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2
OPS = ("fwd", "fwd", "dgrad", "wgrad")


def _cases(count=36, seed=20261202, max_work=2.5e10):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        b = int(rng.integers(1, 25))
        n = 8 * int(rng.integers(1, 401))
        k = 8 * int(rng.integers(1, 401))
        ms = (rng.integers(0, 1600, size=b) * (rng.random(b) > 0.15)).astype(np.int64)
        if ms.sum() == 0:
            ms[0] = int(rng.integers(1, 600))
        while int(ms.sum()) * n * k > max_work:
            ms //= 2
        cases.append((i, OPS[i % len(OPS)], int(rng.integers(0, 2)), b, n, k, [int(v) for v in ms],
                      i % 3 == 0))
    return cases


CASES = _cases()


def _check(got, ref, what):
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    got = got.float()
    assert not torch.isnan(got).any(), f"{what}: unwritten (NaN) outputs"
    err = (got - ref).abs()
    bad = int((err > ATOL + RTOL * ref.abs()).sum())
    assert bad == 0, f"{what}: {bad}/{got.numel()} outputs off, max err {float(err.max())}"


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}" for c in CASES])
def test_random_shape(pkg, monkeypatch, case):
    monkeypatch.delenv("GG_SMALL", raising=False)  # the planner's own choice, small tiles included
    i, op, dt, b, n, k, ms, device_sizes = case
    print(f"[random] case {i}: {op} {'fp16' if dt else 'bf16'} B={b} N={n} K={k} rows={sum(ms)} "
          f"device_sizes={device_sizes}", flush=True)
    td = torch.float16 if dt else torch.bfloat16
    gen = torch.Generator(device=DEV).manual_seed(1000 + i)
    tot = sum(ms)
    gm = torch.tensor(ms, dtype=torch.int64, device=DEV) if device_sizes else ms
    offs = np.concatenate([[0], np.cumsum(ms)])
    if op == "fwd":
        x = torch.randn((tot, k), generator=gen, device=DEV).to(td)
        w = torch.randn((b, n, k), generator=gen, device=DEV).to(td)
        out = torch.full((tot, n), float("nan"), dtype=td, device=DEV)
        pkg.grouped_gemm(x, w, gm, out=out)
        torch.cuda.synchronize(DEV)
        for g in range(b):
            r0, r1 = int(offs[g]), int(offs[g + 1])
            if r1 > r0:
                ref = x[r0:r1].float() @ w[g].float().t().contiguous()
                _check(out[r0:r1], ref, f"case {i} group {g}")
    elif op == "dgrad":
        go = torch.randn((tot, n), generator=gen, device=DEV).to(td)
        w = torch.randn((b, n, k), generator=gen, device=DEV).to(td)
        out = torch.full((tot, k), float("nan"), dtype=td, device=DEV)
        pkg.grouped_gemm_dgrad(go, w, gm, out=out)
        torch.cuda.synchronize(DEV)
        for g in range(b):
            r0, r1 = int(offs[g]), int(offs[g + 1])
            if r1 > r0:
                _check(out[r0:r1], go[r0:r1].float() @ w[g].float(), f"case {i} group {g}")
    else:
        go = torch.randn((tot, n), generator=gen, device=DEV).to(td)
        x = torch.randn((tot, k), generator=gen, device=DEV).to(td)
        out = torch.full((b, n, k), float("nan"), dtype=td, device=DEV)
        pkg.grouped_gemm_wgrad(go, x, gm, out=out)
        torch.cuda.synchronize(DEV)
        for g in range(b):
            r0, r1 = int(offs[g]), int(offs[g + 1])
            ref = go[r0:r1].float().t().contiguous() @ x[r0:r1].float()
            _check(out[g], ref, f"case {i} group {g}")


F8 = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}
# (pass, format of x / grad_out, format of w / x): the recipes the library takes
F8_RECIPES = (("fwd", 0, 0), ("fwd", 1, 1), ("dgrad", 1, 0), ("wgrad", 1, 0), ("dgrad", 0, 0), ("wgrad", 1, 1))


def _cases_fp8(count=12, seed=20261203, max_work=2.0e10):
    rng = np.random.default_rng(seed)
    out = []
    for i, (op, fa, fb) in enumerate(F8_RECIPES * (count // len(F8_RECIPES))):
        b = int(rng.integers(1, 17))
        n = 16 * int(rng.integers(1, 201))  # fp8 rows of 16-byte chunks: N and K multiples of 16
        k = 16 * int(rng.integers(1, 201))
        ms = (rng.integers(0, 1600, size=b) * (rng.random(b) > 0.15)).astype(np.int64)
        if ms.sum() == 0:
            ms[0] = int(rng.integers(1, 600))
        while int(ms.sum()) * n * k > max_work:
            ms //= 2
        out.append((i, op, fa, fb, b, n, k, [int(v) for v in ms], op != "fwd" and i % 2 == 1))
    return out


CASES_FP8 = _cases_fp8()


@pytest.mark.parametrize("case", CASES_FP8, ids=[f"{c[0]}-{c[1]}" for c in CASES_FP8])
def test_random_shape_fp8(pkg, case):
    """fp8 operands, bf16 outputs scaled by the tensor-wise scales: every output against the fp32
    product of the decoded operands times the scales."""
    i, op, fa, fb, b, n, k, ms, device_sizes = case
    print(f"[random fp8] case {i}: {op} formats {fa}/{fb} B={b} N={n} K={k} rows={sum(ms)} "
          f"device_sizes={device_sizes}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(5000 + i)
    tot = sum(ms)
    gm = torch.tensor(ms, dtype=torch.int64, device=DEV) if device_sizes else ms
    offs = np.concatenate([[0], np.cumsum(ms)])
    s_a = (torch.rand(1, generator=gen, device=DEV) * 1.5 + 0.5).float()
    s_b = (torch.rand(b, generator=gen, device=DEV) * 1.5 + 0.5).float()
    if op == "fwd":
        x = torch.randn((tot, k), generator=gen, device=DEV).to(F8[fa])
        w = torch.randn((b, n, k), generator=gen, device=DEV).to(F8[fb])
        out = torch.full((tot, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        pkg.grouped_gemm_fp8(x, w, gm, s_a, s_b, out=out)
        torch.cuda.synchronize(DEV)
        for g in range(b):
            r0, r1 = int(offs[g]), int(offs[g + 1])
            if r1 > r0:
                ref = (x[r0:r1].float() @ w[g].float().t().contiguous()) * (s_a[0] * s_b[g])
                _check(out[r0:r1], ref, f"case {i} group {g}")
    elif op == "dgrad":
        go = torch.randn((tot, n), generator=gen, device=DEV).to(F8[fa])
        w = torch.randn((b, n, k), generator=gen, device=DEV).to(F8[fb])
        out = torch.full((tot, k), float("nan"), dtype=torch.bfloat16, device=DEV)
        pkg.grouped_gemm_dgrad_fp8(go, w, gm, s_a, s_b, out=out)
        torch.cuda.synchronize(DEV)
        for g in range(b):
            r0, r1 = int(offs[g]), int(offs[g + 1])
            if r1 > r0:
                _check(out[r0:r1], (go[r0:r1].float() @ w[g].float()) * (s_a[0] * s_b[g]), f"case {i} group {g}")
    else:
        go = torch.randn((tot, n), generator=gen, device=DEV).to(F8[fa])
        x = torch.randn((tot, k), generator=gen, device=DEV).to(F8[fb])
        out = torch.full((b, n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
        pkg.grouped_gemm_wgrad_fp8(go, x, gm, s_a, s_b, out=out)
        torch.cuda.synchronize(DEV)
        for g in range(b):
            r0, r1 = int(offs[g]), int(offs[g + 1])
            ref = (go[r0:r1].float().t().contiguous() @ x[r0:r1].float()) * (s_a[0] * s_b[g])
            _check(out[g], ref, f"case {i} group {g}")
