"""Partial tiles on the GPU: every residue of a tile's valid rows and columns, in every layout.

The waves of a K-major A take interleaved 16-row blocks (wave wm's block mi is tile rows
16 (2 mi + wm) ..), and in the cross-tile variant a tile with at most 128 valid rows (or a wave
whose columns are all past N) skips the MFMAs of its row blocks that hold no valid output (thin
K steps). These tests cover the row counts 1 .. 256 at every residue mod 32 (both waves' shares,
a wave with no block at all), column tails of 8 .. 248, and both kernel variants (per-tile: one
tile per workgroup, every block computed; cross-tile: several tiles per workgroup, where a
partial tile's stale accumulators must never reach the next tile's stores), for the forward,
dgrad, wgrad, fp8, split-K and device-size paths.

Bar: every output within rtol = atol = 1e-2 of a float32 product of the same inputs
(bench/bench_main.cpp:264-268); outputs are NaN-prefilled, so a row or column left unwritten,
or written with a stale accumulator, fails.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2


def _rand(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV, dtype=torch.float32).to(dtype)


def _check(got, ref, what):
    got = got.float()
    assert not torch.isnan(got).any(), f"{what}: unwritten outputs"
    err = (got - ref).abs()
    bad = int((err > ATOL + RTOL * ref.abs()).sum())
    assert bad == 0, f"{what}: {bad}/{got.numel()} outputs off, max err {float(err.max())}"


def _fwd_ref(x, w, gm, scale=None):
    outs, row = [], 0
    for g, m in enumerate(gm):
        r = x[row:row + m].float() @ w[g].float().t().contiguous()
        if scale is not None:
            r = r * scale[g]
        outs.append(r)
        row += m
    return torch.cat(outs) if outs else torch.empty(0, w.shape[1], device=DEV)


# row counts at every residue mod 32 within one tile, and across a tile boundary
ROWS_ONE_TILE = [1, 8, 15, 16, 17, 31, 32, 33, 48, 63, 100, 127, 128, 129, 144, 160, 200, 224, 240, 255, 256]
ROWS_MULTI = [16 * i + (i % 16) + 1 for i in range(40)]  # 1 .. 664 rows, every residue mod 16


@pytest.mark.parametrize("n", [8, 136, 264, 248])
def test_forward_per_tile_rows_and_columns(pkg, n):
    gm, k = ROWS_ONE_TILE, 136  # one M-tile per group, K % 64 = 8
    print(f"[tails] forward per-tile: N={n} K={k} group_m={gm}", flush=True)
    x, w = _rand((sum(gm), k), 1), _rand((len(gm), n, k), 2)
    out = torch.full((sum(gm), n), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm(x, w, gm, out=out)
    _check(out, _fwd_ref(x, w, gm), f"forward N={n}")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_forward_cross_tile_ragged(pkg, dt):
    gm, n, k = ROWS_MULTI, 2056, 320  # 9 N-tiles (last one 8 columns), > 256 tiles, 5 K steps
    print(f"[tails] forward cross-tile: dtype={dt} N={n} K={k} groups={len(gm)}", flush=True)
    x, w = _rand((sum(gm), k), 3, dt), _rand((len(gm), n, k), 4, dt)
    out = torch.full((sum(gm), n), float("nan"), dtype=dt, device=DEV)
    pkg.grouped_gemm(x, w, gm, out=out)
    _check(out, _fwd_ref(x, w, gm), "forward cross-tile")


def test_forward_device_sizes_ragged(pkg):
    gm, n, k = ROWS_MULTI[:24], 1160, 448
    print(f"[tails] forward device sizes: N={n} K={k} groups={len(gm)}", flush=True)
    x, w = _rand((sum(gm), k), 5), _rand((len(gm), n, k), 6)
    out = torch.full((sum(gm), n), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm(x, w, torch.tensor(gm, dtype=torch.int64, device=DEV), out=out)
    _check(out, _fwd_ref(x, w, gm), "forward device sizes")


@pytest.mark.parametrize("sp", [2, 5])
def test_forward_split_k_tails(pkg, monkeypatch, sp):
    monkeypatch.setenv("GG_SPLIT_K", str(sp))
    gm, n, k = [129, 255, 17], 264, 1088
    print(f"[tails] forward split-K S={sp}: group_m={gm} N={n} K={k}", flush=True)
    x, w = _rand((sum(gm), k), 7), _rand((len(gm), n, k), 8)
    out = torch.full((sum(gm), n), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm(x, w, gm, out=out)
    _check(out, _fwd_ref(x, w, gm), f"split-K {sp}")


@pytest.mark.parametrize("gm,n,k", [(ROWS_ONE_TILE, 264, 200), (ROWS_MULTI, 1032, 2056)])
def test_dgrad_tails(pkg, gm, n, k):
    # grad_x [sum(M), K] = grad_out [sum(M), N] @ w[g] [N, K]: output rows are the group's rows
    print(f"[tails] dgrad: N={n} K={k} groups={len(gm)}", flush=True)
    go, w = _rand((sum(gm), n), 9), _rand((len(gm), n, k), 10)
    out = torch.full((sum(gm), k), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm_dgrad(go, w, gm, out=out)
    refs, row = [], 0
    for g, m in enumerate(gm):
        refs.append(go[row:row + m].float() @ w[g].float())
        row += m
    _check(out, torch.cat(refs), "dgrad")


@pytest.mark.parametrize("n,k", [(8, 264), (136, 1000), (1000, 136), (2056, 520)])
def test_wgrad_tails(pkg, n, k):
    # grad_w [B, N, K] = grad_out[g]^T [N, M] @ x[g] [M, K]: output rows are N (contiguous row
    # blocks, the MN-major A), columns K
    gm = [300, 517, 64, 1]
    print(f"[tails] wgrad: N={n} K={k} group_m={gm}", flush=True)
    go, x = _rand((sum(gm), n), 11), _rand((sum(gm), k), 12)
    out = torch.full((len(gm), n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm_wgrad(go, x, gm, out=out)
    row = 0
    for g, m in enumerate(gm):
        ref = go[row:row + m].float().t().contiguous() @ x[row:row + m].float()
        _check(out[g], ref, f"wgrad group {g}")
        row += m


@pytest.mark.parametrize("fdt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_fp8_forward_tails(pkg, fdt):
    gm, n, k = ROWS_MULTI[:30], 1160, 384
    print(f"[tails] fp8 forward {fdt}: N={n} K={k} groups={len(gm)}", flush=True)
    x, w = _rand((sum(gm), k), 13).to(fdt), _rand((len(gm), n, k), 14).to(fdt)
    xs = torch.tensor([0.5], dtype=torch.float32, device=DEV)
    ws = torch.linspace(0.25, 2.0, len(gm), dtype=torch.float32, device=DEV)
    out = torch.full((sum(gm), n), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm_fp8(x, w, gm, xs, ws, out=out)
    _check(out, _fwd_ref(x, w, gm, scale=(ws * xs).tolist()), "fp8 forward")


def test_fp8_dgrad_tails(pkg):
    gm, n, k = ROWS_ONE_TILE, 272, 400  # fp8 backward: N, K multiples of 16
    print(f"[tails] fp8 dgrad: N={n} K={k} groups={len(gm)}", flush=True)
    go = _rand((sum(gm), n), 15).to(torch.float8_e5m2)
    w = _rand((len(gm), n, k), 16).to(torch.float8_e4m3fn)
    gs = torch.tensor([1.0], dtype=torch.float32, device=DEV)
    wsc = torch.ones(len(gm), dtype=torch.float32, device=DEV)
    out = torch.full((sum(gm), k), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.grouped_gemm_dgrad_fp8(go, w, gm, gs, wsc, out=out)
    refs, row = [], 0
    for g, m in enumerate(gm):
        refs.append(go[row:row + m].float() @ w[g].float())
        row += m
    _check(out, torch.cat(refs), "fp8 dgrad")


def _run_plan(pkg, kind, dt, n, k, gm, go, other, out, **kw):
    s = torch.cuda.current_stream(DEV).cuda_stream
    plan = pkg.BackwardPlan(kind, dt, n, k, gm, go.data_ptr(), other.data_ptr(), out.data_ptr(), s, **kw)
    plan.run(s)
    torch.cuda.synchronize(DEV)
    detail = plan.detail()
    plan.release()
    return detail


def test_wgrad_cross_tile_tails(pkg):
    # > 256 tiles and every group >= 4 K steps of 64 rows: the cross-tile variant, with a 8-row
    # tail (N = 2056 output rows, contiguous row blocks) and an 8-column tail (K = 2056)
    gm, n, k = [300, 517, 640, 1000], 2056, 2056
    print(f"[tails] wgrad cross-tile: N={n} K={k} group_m={gm}", flush=True)
    go, x = _rand((sum(gm), n), 17), _rand((sum(gm), k), 18)
    out = torch.full((len(gm), n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
    detail = _run_plan(pkg, "wgrad", pkg.DType.BF16, n, k, gm, go, x, out)
    assert "cross-tile" in detail, detail
    row = 0
    for g, m in enumerate(gm):
        ref = go[row:row + m].float().t().contiguous() @ x[row:row + m].float()
        _check(out[g], ref, f"wgrad cross-tile group {g}")
        row += m


def test_fp8_wgrad_cross_tile_tails(pkg):
    # fp8 K steps are 128 rows: every group >= 4 steps; N = K = 2064 (16-row and 16-column tails)
    gm, n, k = [600, 1000, 513, 1400], 2064, 2064
    print(f"[tails] fp8 wgrad cross-tile: N={n} K={k} group_m={gm}", flush=True)
    go = _rand((sum(gm), n), 19).to(torch.float8_e5m2)
    x = _rand((sum(gm), k), 20).to(torch.float8_e4m3fn)
    gs = torch.tensor([0.5], dtype=torch.float32, device=DEV)
    xs = torch.linspace(0.5, 1.5, len(gm), dtype=torch.float32, device=DEV)
    out = torch.full((len(gm), n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
    detail = _run_plan(pkg, "wgrad", pkg.DType.FP8_E5M2, n, k, gm, go, x, out, other_dtype=pkg.DType.FP8_E4M3,
                       grad_scale=gs.data_ptr(), other_scale=xs.data_ptr())
    assert "cross-tile" in detail, detail
    row = 0
    for g, m in enumerate(gm):
        ref = (go[row:row + m].float().t().contiguous() @ x[row:row + m].float()) * (0.5 * float(xs[g]))
        _check(out[g], ref, f"fp8 wgrad cross-tile group {g}")
        row += m
