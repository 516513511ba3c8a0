"""gg_run_device_lens_noalloc: the allocation-free call, through the C ABI on the GPU.

Bar: the same bits as a gg_prepare_device_lens_op plan + gg_run on the same inputs (both use the
same kernels; only where the group table lives differs), on two calls in a row with the second
one smaller, so that the scratch array holds the first call's table when the second starts.
Every output is also checked against torch fp32 within rtol = atol = 1e-2
(bench/bench_main.cpp:264-268).
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


def _case(pkg, b, n, k, lens, gap=0, seed=7):
    """x, w, device lens and offsets (gap empty rows before every group), and total rows."""
    lens = [int(v) for v in lens]
    offs, row = [], 0
    for m in lens:
        row += gap
        offs.append(row)
        row += m
    offs.append(row)
    total = row
    x = torch.empty((total, k), dtype=torch.bfloat16, device=DEV)
    w = torch.empty((b, n, k), dtype=torch.bfloat16, device=DEV)
    pkg.fill_randn(pkg.DType.BF16, x.data_ptr(), x.numel(), seed, _stream())
    pkg.fill_randn(pkg.DType.BF16, w.data_ptr(), w.numel(), seed + 1, _stream())
    d_lens = torch.tensor(lens, dtype=torch.int64, device=DEV)
    d_offs = torch.tensor(offs, dtype=torch.int64, device=DEV)
    return x, w, d_lens, d_offs, offs, total


def _planned(pkg, x, w, d_lens, d_offs, total):
    b, n, k = w.shape
    out = torch.full((total, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    plan = pkg.DeviceLensPlan(pkg.OP_FORWARD, pkg.DType.BF16, pkg.DType.BF16, b, total, n, k, d_lens.data_ptr(),
                              d_offs.data_ptr(), x.data_ptr(), w.data_ptr(), out.data_ptr(), _stream())
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    plan.release()
    return out


def _noalloc(pkg, x, w, d_lens, d_offs, total):
    b, n, k = w.shape
    out = torch.full((total, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.run_device_lens_noalloc(pkg.OP_FORWARD, pkg.DType.BF16, pkg.DType.BF16, b, total, n, k, d_lens.data_ptr(),
                                d_offs.data_ptr(), x.data_ptr(), w.data_ptr(), out.data_ptr(), _stream())
    torch.cuda.synchronize(DEV)
    return out


def _torch_ref(x, w, offs, lens):
    b, n, _ = w.shape
    ref = torch.full((x.shape[0], n), float("nan"), dtype=torch.float32, device=DEV)
    for g in range(b):
        r0, m = offs[g], lens[g]
        if m:
            ref[r0:r0 + m] = x[r0:r0 + m].float() @ w[g].float().t()
    return ref


def _check(pkg, b, n, k, lens, gap):
    print(f"[no_alloc] B={b} N={n} K={k} rows={sum(lens)} gap={gap}", flush=True)
    x, w, d_lens, d_offs, offs, total = _case(pkg, b, n, k, lens, gap)
    got = _noalloc(pkg, x, w, d_lens, d_offs, total)
    want = _planned(pkg, x, w, d_lens, d_offs, total)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "not the bits of the planned run"
    ref = _torch_ref(x, w, offs, lens)
    written = ~torch.isnan(ref)
    assert torch.equal(~torch.isnan(got.float()), written), "rows outside the groups were written"
    diff = (got.float() - ref).abs()[written]
    tol = (ATOL + RTOL * ref.abs())[written]
    assert bool((diff <= tol).all()), f"max abs err {diff.max().item()}"


def test_two_calls_in_a_row_second_smaller(pkg):
    rng = np.random.default_rng(11)
    # 80 groups: more than the in-kernel table holds, so the table kernel writes it into scratch;
    # some groups are empty, and empty rows sit between groups
    lens1 = rng.integers(0, 300, size=80)
    lens1[[3, 40, 79]] = 0
    _check(pkg, 80, 512, 384, lens1, gap=5)
    # then a smaller call: 6 groups (the GEMM builds the table, writes the header in scratch)
    lens2 = rng.integers(1, 200, size=6)
    _check(pkg, 6, 256, 136, lens2, gap=0)


def test_empty_contraction_zero_fills(pkg):
    x, w, d_lens, d_offs, _, total = _case(pkg, 3, 64, 8, [17, 0, 40])
    out = torch.full((total, 64), float("nan"), dtype=torch.bfloat16, device=DEV)
    pkg.run_device_lens_noalloc(pkg.OP_FORWARD, pkg.DType.BF16, pkg.DType.BF16, 3, total, 64, 0, d_lens.data_ptr(),
                                d_offs.data_ptr(), x.data_ptr(), w.data_ptr(), out.data_ptr(), _stream())
    torch.cuda.synchronize(DEV)
    assert bool((out == 0).all())


def test_too_many_groups_is_refused(pkg):
    lens = torch.zeros(8193, dtype=torch.int64, device=DEV)
    x = torch.empty((8, 64), dtype=torch.bfloat16, device=DEV)
    w = torch.empty((1, 64, 64), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((8, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(pkg.GGError) as e:
        pkg.run_device_lens_noalloc(pkg.OP_FORWARD, pkg.DType.BF16, pkg.DType.BF16, 8193, 8, 64, 64,
                                    lens.data_ptr(), 0, x.data_ptr(), w.data_ptr(), out.data_ptr(), _stream())
    assert "at most 8192 groups" in str(e.value)


def test_wgrad_more_than_64_groups(pkg):
    """wgrad through the scratch table with more than 64 groups (the table kernel writes its
    out_rows-based tiles into scratch): the planned path's bits and torch fp32, on two calls in a
    row, the second smaller."""
    rng = np.random.default_rng(21)
    for b, n, k in ((72, 256, 192), (66, 128, 64)):
        lens = rng.integers(0, 200, size=b)
        lens[[1, b - 1]] = 0
        total = int(lens.sum())
        print(f"[no_alloc] wgrad B={b} N={n} K={k} rows={total}", flush=True)
        go = torch.randn((total, n), device=DEV).to(torch.bfloat16)
        x = torch.randn((total, k), device=DEV).to(torch.bfloat16)
        d_lens = torch.tensor(lens, dtype=torch.int64, device=DEV)
        want = torch.full((b, n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
        plan = pkg.DeviceLensPlan(pkg.OP_WGRAD, pkg.DType.BF16, pkg.DType.BF16, b, total, n, k, d_lens.data_ptr(), 0,
                                  go.data_ptr(), x.data_ptr(), want.data_ptr(), _stream())
        plan.run(_stream())
        torch.cuda.synchronize(DEV)
        plan.release()
        got = torch.full((b, n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
        pkg.run_device_lens_noalloc(pkg.OP_WGRAD, pkg.DType.BF16, pkg.DType.BF16, b, total, n, k, d_lens.data_ptr(),
                                    0, go.data_ptr(), x.data_ptr(), got.data_ptr(), _stream())
        torch.cuda.synchronize(DEV)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "not the bits of the planned run"
        row = 0
        for g, m in enumerate(int(v) for v in lens):
            ref = go[row:row + m].float().t().contiguous() @ x[row:row + m].float()
            row += m
            assert bool(((got[g].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()), f"group {g}"


@pytest.mark.parametrize("b", [6, 70])
def test_graph_capture_replays(pkg, b):
    """One call outside capture (it sets up the device's scratch address), then the call captured
    in a CUDA graph (6 groups: one launch, the GEMM builds the table; 70: the table kernel and the
    GEMM) and replayed three times, with eager work and synchronizations between the replays:
    every replay gives the planned path's bits."""
    rng = np.random.default_rng(31 + b)
    lens = rng.integers(0, 300, size=b)
    lens[0] = 0
    n, k = 384, 200
    print(f"[no_alloc] graph B={b} N={n} K={k} rows={int(lens.sum())}", flush=True)
    x, w, d_lens, d_offs, offs, total = _case(pkg, b, n, k, lens, gap=3)
    want = _planned(pkg, x, w, d_lens, d_offs, total)
    first = _noalloc(pkg, x, w, d_lens, d_offs, total)
    assert torch.equal(first.view(torch.int16), want.view(torch.int16))
    out = torch.full((total, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize(DEV)
    with torch.cuda.graph(graph):
        pkg.run_device_lens_noalloc(pkg.OP_FORWARD, pkg.DType.BF16, pkg.DType.BF16, b, total, n, k,
                                    d_lens.data_ptr(), d_offs.data_ptr(), x.data_ptr(), w.data_ptr(), out.data_ptr(),
                                    torch.cuda.current_stream(DEV).cuda_stream)
    sx, sw, s_lens, s_offs, _, s_total = _case(pkg, 1, 64, 64, [5], seed=3)
    for replay in range(3):
        out.fill_(float("nan"))
        _noalloc(pkg, sx, sw, s_lens, s_offs, s_total)  # another call on the scratch between replays
        torch.cuda.synchronize(DEV)
        graph.replay()
        torch.cuda.synchronize(DEV)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {replay}"
