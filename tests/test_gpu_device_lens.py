"""Device-resident group sizes (gg_prepare_device_lens), through the C ABI on the GPU.

The sizes are a device int64 tensor, as MoE routing produces them and as the reference's
vendored Primus-Turbo grouped GEMM takes them (grouped_gemm.h:35-36, 95-96: group_lens_ptr,
group_offs_ptr). Bar: the same bits as a plan built from the same sizes on the host, every output
within rtol = atol = 1e-2 of fp32 (bench/bench_main.cpp:264-268), rows outside every group left
untouched, and sizes that do not fit reported, never written.
"""
import os

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


def _inputs(pkg, dt, rows, b, n, k, seed_x=1, seed_w=2):
    td = torch.bfloat16 if dt == 0 else torch.float16
    x = torch.empty((rows, k), dtype=td, device=DEV)
    w = torch.empty((b, n, k), dtype=td, device=DEV)
    pkg.fill_randn(pkg.DType(dt), x.data_ptr(), x.numel(), seed_x, _stream())
    pkg.fill_randn(pkg.DType(dt), w.data_ptr(), w.numel(), seed_w, _stream())
    return x, w


def _host_plan_out(pkg, dt, x, w, group_m):
    """Output of the host-size plan (gg_prepare) on the same inputs, NaN where unwritten. Split-K
    off, as in a device-size plan (whose tile count is unknown on the host), so that every
    output has the same fp32 summation order in both."""
    b, n, k = w.shape
    out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device=DEV)
    be = pkg.make_mi355x_backend()
    prob = pkg.GroupedGemmProblem(pkg.DType(dt), b, n, k, list(group_m), x.data_ptr(), w.data_ptr(),
                                  out.data_ptr())
    old = os.environ.get("GG_SPLIT_K")
    os.environ["GG_SPLIT_K"] = "1"
    try:
        assert be.prepare(prob, _stream()) == ""
    finally:
        if old is None:
            del os.environ["GG_SPLIT_K"]
        else:
            os.environ["GG_SPLIT_K"] = old
    be.run(_stream())
    torch.cuda.synchronize(DEV)
    be.release()
    return out


class DevicePlan:
    """A gg_prepare_device_lens plan over device lens/offs tensors, reusable across runs."""

    def __init__(self, pkg, dt, x, w, lens, offs=None, total_m=None):
        self.pkg, self.x, self.w, self.lens, self.offs = pkg, x, w, lens, offs
        b, n, k = w.shape
        self.out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device=DEV)
        self.be = pkg.make_mi355x_backend()
        why = self.be.prepare_device_lens(pkg.DType(dt), b, x.shape[0] if total_m is None else total_m,
                                          n, k, lens.data_ptr(), offs.data_ptr() if offs is not None else 0,
                                          x.data_ptr(), w.data_ptr(), self.out.data_ptr(), _stream())
        assert why == "", why

    def run(self):
        self.be.run(_stream())
        st, tiles, msg = self.be.device_status(_stream())
        return st, tiles, msg

    def close(self):
        self.be.release()


def _check_group(x, w, out, g, row0, m):
    ref = x[row0:row0 + m].float() @ w[g].float().t().contiguous()
    got = out[row0:row0 + m].float()
    assert not torch.isnan(got).any(), f"group {g}: unwritten outputs"
    bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
    assert bad == 0, f"group {g}: {bad} outputs off"


CASES = [
    (0, [520] * 6, 2880, 2880),                 # 5a-like: M and N tails, several tiles per workgroup
    (0, [3000, 0, 17, 900, 0, 4100], 776, 1216),  # unbalanced routing with empty experts
    (1, [1, 255, 257, 0], 264, 128),            # fp16, off-by-one rows, short K (per-tile path)
    (0, [0, 0, 0], 512, 512),                   # no tokens routed at all
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_device_sizes_match_host_sizes(pkg, case):
    dt, gm, n, k = CASES[case]
    print(f"[device-lens] case {case}: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    rows = max(1, sum(gm))
    x, w = _inputs(pkg, dt, rows, len(gm), n, k)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    plan = DevicePlan(pkg, dt, x, w, lens)
    st, tiles, msg = plan.run()
    assert st == pkg.GG_OK, msg
    host = _host_plan_out(pkg, dt, x, w, gm)
    ntile = -(-n // 256)
    assert tiles == sum(-(-m // 256) * ntile for m in gm)
    if sum(gm) > 0:
        assert torch.equal(plan.out.view(torch.int16), host.view(torch.int16)), "bits differ from host plan"
    row = 0
    for g, m in enumerate(gm):
        if m:
            _check_group(x, w, plan.out, g, row, m)
        row += m
    plan.close()


def test_offsets_leave_gaps_untouched(pkg, oracle):
    """group_offs places groups with gaps between them (padded routing buffers): rows in the gaps
    are not written; every group matches the oracle on the reference driver's samples."""
    gm, starts, n, k = [300, 0, 777, 64], [16, 400, 512, 1400], 1032, 640
    total = 1500
    x, w = _inputs(pkg, 0, total, len(gm), n, k)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    offs = torch.tensor(starts + [total], dtype=torch.int64, device=DEV)
    plan = DevicePlan(pkg, 0, x, w, lens, offs)
    st, _, msg = plan.run()
    assert st == pkg.GG_OK, msg
    written = torch.zeros(total, dtype=torch.bool)
    for g, (r0, m) in enumerate(zip(starts, gm)):
        if m:
            _check_group(x, w, plan.out, g, r0, m)
            written[r0:r0 + m] = True
    gaps = plan.out[~written.to(DEV)]
    assert torch.isnan(gaps.float()).all(), "rows outside every group were written"
    # the driver's sampled check on the packed groups, against the CPU oracle
    xs = torch.cat([x[r0:r0 + m] for r0, m in zip(starts, gm)])
    outs = torch.cat([plan.out[r0:r0 + m] for r0, m in zip(starts, gm)])
    s = oracle.make_samples(len(gm), n, gm, 256)
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    ref = oracle.sampled(0, bits(xs), bits(w), s)
    got = outs[torch.from_numpy(s[:, 0]).to(DEV), torch.from_numpy(s[:, 1]).to(DEV)].float().cpu().numpy()
    nbad, _ = oracle.check(got, ref, ATOL, RTOL)
    assert nbad == 0
    plan.close()


def test_one_plan_serves_changing_routing(pkg):
    """The plan is built once; the sizes change on the device between runs (a new routing per
    step), with no host read and no new plan. Each run matches a host plan of its sizes."""
    n, k, b, total = 1024, 1024, 4, 4096
    x, w = _inputs(pkg, 0, total, b, n, k)
    lens = torch.zeros(b, dtype=torch.int64, device=DEV)
    plan = DevicePlan(pkg, 0, x, w, lens)
    for routing in ([1024] * 4, [4096, 0, 0, 0], [7, 1500, 2000, 589], [0, 0, 0, 0], [100, 3000, 0, 996]):
        lens.copy_(torch.tensor(routing, dtype=torch.int64))
        plan.out.fill_(float("nan"))
        st, _, msg = plan.run()
        assert st == pkg.GG_OK, msg
        host = _host_plan_out(pkg, 0, x, w, routing)
        used = sum(routing)
        assert torch.equal(plan.out[:used].view(torch.int16), host[:used].view(torch.int16)), routing
        assert torch.isnan(plan.out[used:].float()).all(), routing
    plan.close()


def test_sizes_that_do_not_fit_are_reported_not_written(pkg):
    """A negative length, or rows past total_m, gives that group no work and a status naming it;
    the groups before it are computed normally."""
    n, k = 512, 256
    x, w = _inputs(pkg, 0, 1000, 3, n, k)
    # back to back: group 2 would end at row 1100 > 1000
    lens = torch.tensor([300, 500, 300], dtype=torch.int64, device=DEV)
    plan = DevicePlan(pkg, 0, x, w, lens)
    st, _, msg = plan.run()
    assert st == pkg.GG_ERR_INVALID and "group 2" in msg, msg
    _check_group(x, w, plan.out, 0, 0, 300)
    _check_group(x, w, plan.out, 1, 300, 500)
    assert torch.isnan(plan.out[800:].float()).all()
    plan.close()
    # a negative length
    lens = torch.tensor([300, -5, 200], dtype=torch.int64, device=DEV)
    plan = DevicePlan(pkg, 0, x, w, lens)
    st, _, msg = plan.run()
    assert st == pkg.GG_ERR_INVALID and "group 1" in msg, msg
    _check_group(x, w, plan.out, 0, 0, 300)
    _check_group(x, w, plan.out, 2, 300, 200)
    plan.close()
    # an offset before row 0
    lens = torch.tensor([100, 100, 100], dtype=torch.int64, device=DEV)
    offs = torch.tensor([0, -50, 500, 1000], dtype=torch.int64, device=DEV)
    plan = DevicePlan(pkg, 0, x, w, lens, offs)
    st, _, msg = plan.run()
    assert st == pkg.GG_ERR_INVALID and "group 1" in msg, msg
    _check_group(x, w, plan.out, 0, 0, 100)
    _check_group(x, w, plan.out, 2, 500, 100)
    plan.close()


def test_torch_wrapper_takes_device_sizes(pkg):
    """grouped_gemm(x, w, group_m) with group_m a device tensor (the routing output)."""
    gm = [700, 0, 1324]
    x, w = _inputs(pkg, 1, sum(gm), len(gm), 776, 520)
    out = pkg.grouped_gemm(x, w, torch.tensor(gm, dtype=torch.int64, device=DEV))
    row = 0
    for g, m in enumerate(gm):
        if m:
            _check_group(x, w, out, g, row, m)
        row += m
    with pytest.raises(pkg.GGError):
        pkg.grouped_gemm(x, w, torch.tensor([700, 0, 2000], dtype=torch.int64, device=DEV))


@pytest.mark.parametrize("b", [1, 8, 63, 64, 65, 300])
def test_compute_group_offs(pkg, b):
    """offs = [0, cumsum(lens)] on the device, across the 64-group chunks of the scan."""
    gen = torch.Generator().manual_seed(b)
    lens = torch.randint(0, 5000, (b,), generator=gen, dtype=torch.int64)
    lens[::7] = 0
    offs = pkg.compute_group_offs(lens.to(DEV))
    torch.cuda.synchronize(DEV)
    want = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lens, 0)])
    assert torch.equal(offs.cpu(), want)


# ---- every pass over device sizes (gg_prepare_device_lens_op) --------------------------------
TDT8 = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}


def _dt8(pkg, f):
    return pkg.DType.FP8_E4M3 if f == 0 else pkg.DType.FP8_E5M2


def _host_backward(pkg, kind, fmts, gm, n, k, go, other, gs=None, os_=None):
    """Output of the host-size backward plan, split-K off, NaN where unwritten."""
    shape = (go.shape[0], k) if kind == "dgrad" else (len(gm), n, k)
    odt = torch.bfloat16 if fmts is not None else go.dtype
    out = torch.full(shape, float("nan"), dtype=odt, device=DEV)
    old = os.environ.get("GG_SPLIT_K")
    os.environ["GG_SPLIT_K"] = "1"
    try:
        if fmts is None:
            dt = pkg.DType.BF16 if go.dtype == torch.bfloat16 else pkg.DType.FP16
            plan = pkg.BackwardPlan(kind, dt, n, k, gm, go.data_ptr(), other.data_ptr(), out.data_ptr(), _stream())
        else:
            plan = pkg.BackwardPlan(kind, _dt8(pkg, fmts[0]), n, k, gm, go.data_ptr(), other.data_ptr(),
                                    out.data_ptr(), _stream(), other_dtype=_dt8(pkg, fmts[1]),
                                    grad_scale=gs.data_ptr(), other_scale=os_.data_ptr())
    finally:
        if old is None:
            del os.environ["GG_SPLIT_K"]
        else:
            os.environ["GG_SPLIT_K"] = old
    plan.run(_stream())
    torch.cuda.synchronize(DEV)
    plan.release()
    return out


BWD_CASES = [
    ("dgrad", None, [300, 0, 17, 513], 272, 528),
    ("wgrad", None, [300, 0, 17, 513], 272, 528),
    ("dgrad", None, [1000, 2000, 1100], 1024, 2048),   # more tiles than workgroups (cross-tile)
    ("wgrad", None, [600, 1000, 513, 1400], 1024, 2304),
    ("dgrad", (1, 0), [300, 0, 17, 513], 272, 528),
    ("wgrad", (1, 0), [600, 0, 513, 1400], 1024, 2304),
    ("dgrad", (0, 0), [1000, 2000, 1100], 1024, 2048),
]


@pytest.mark.parametrize("case", range(len(BWD_CASES)))
def test_device_sizes_backward_match_host_sizes(pkg, case):
    """dgrad / wgrad (16-bit and fp8) with device group sizes give the bits of the host-size
    plan on the same inputs; wgrad of an empty group is zero."""
    kind, fmts, gm, n, k = BWD_CASES[case]
    print(f"[device-lens] backward {case}: {kind} formats={fmts} group_m={gm} N={n} K={k}", flush=True)
    rows = sum(gm)
    gen = torch.Generator().manual_seed(40 + case)
    if fmts is None:
        go = torch.randn((rows, n), generator=gen).to(torch.bfloat16).to(DEV)
        other = torch.randn((len(gm), n, k) if kind == "dgrad" else (rows, k), generator=gen).to(torch.bfloat16).to(DEV)
        gs = os_ = None
        adt = bdt = pkg.DType.BF16
    else:
        go = torch.randn((rows, n), generator=gen).to(TDT8[fmts[0]]).to(DEV)
        other = torch.randn((len(gm), n, k) if kind == "dgrad" else (rows, k), generator=gen).to(TDT8[fmts[1]]).to(DEV)
        gs = torch.tensor([0.5], device=DEV)
        os_ = torch.tensor([0.25 * (g + 1) for g in range(len(gm))], device=DEV)
        adt, bdt = _dt8(pkg, fmts[0]), _dt8(pkg, fmts[1])
    shape = (rows, k) if kind == "dgrad" else (len(gm), n, k)
    out = torch.full(shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    plan = pkg.DeviceLensPlan(pkg.OP_DGRAD if kind == "dgrad" else pkg.OP_WGRAD, adt, bdt, len(gm), rows, n, k,
                              lens.data_ptr(), 0, go.data_ptr(), other.data_ptr(), out.data_ptr(), _stream(),
                              gs.data_ptr() if gs is not None else 0, os_.data_ptr() if os_ is not None else 0)
    plan.run(_stream())
    st, _, msg = plan.status(_stream())
    detail = plan.detail()
    plan.release()
    assert st == pkg.GG_OK, msg
    host = _host_backward(pkg, kind, fmts, gm, n, k, go, other, gs, os_)
    assert torch.equal(out.view(torch.int16), host.view(torch.int16)), f"bits differ from host plan ({detail})"
    if kind == "wgrad":
        for g, m in enumerate(gm):
            if m == 0:
                assert torch.count_nonzero(out[g].float()) == 0


def test_device_sizes_fp8_forward(pkg):
    """The fp8 forward over device sizes gives the bits of the host-size fp8 plan."""
    gm, n, k = [700, 0, 1324, 513], 776, 1040
    gen = torch.Generator().manual_seed(50)
    x = torch.randn((sum(gm), k), generator=gen).to(torch.float8_e4m3fn).to(DEV)
    w = torch.randn((len(gm), n, k), generator=gen).to(torch.float8_e4m3fn).to(DEV)
    xs = torch.tensor([1.5], device=DEV)
    ws = torch.tensor([0.5, 1.0, 2.0, 0.25], device=DEV)
    out = torch.full((sum(gm), n), float("nan"), dtype=torch.bfloat16, device=DEV)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    plan = pkg.DeviceLensPlan(pkg.OP_FORWARD, pkg.DType.FP8_E4M3, pkg.DType.FP8_E4M3, len(gm), sum(gm), n, k,
                              lens.data_ptr(), 0, x.data_ptr(), w.data_ptr(), out.data_ptr(), _stream(),
                              xs.data_ptr(), ws.data_ptr())
    plan.run(_stream())
    st, _, msg = plan.status(_stream())
    plan.release()
    assert st == pkg.GG_OK, msg
    host = torch.full_like(out, float("nan"))
    old = os.environ.get("GG_SPLIT_K")
    os.environ["GG_SPLIT_K"] = "1"
    try:
        hp = pkg.Fp8Plan(pkg.DType.FP8_E4M3, n, k, gm, x.data_ptr(), w.data_ptr(), xs.data_ptr(), ws.data_ptr(),
                         host.data_ptr(), _stream())
    finally:
        if old is None:
            del os.environ["GG_SPLIT_K"]
        else:
            os.environ["GG_SPLIT_K"] = old
    hp.run(_stream())
    torch.cuda.synchronize(DEV)
    hp.release()
    assert torch.equal(out.view(torch.int16), host.view(torch.int16))


def test_device_sizes_backward_bad_sizes_and_wrappers(pkg):
    """A negative length is reported and its group computes nothing (wgrad: zero output); the
    torch wrappers take device sizes."""
    gm, n, k = [300, 500, 200], 512, 256
    go = _inputs(pkg, 0, sum(gm), 1, n, n)[0][:, :n].contiguous()
    x = _inputs(pkg, 0, sum(gm), 1, k, k, seed_x=7)[0][:, :k].contiguous()
    bad = torch.tensor([300, -5, 200], dtype=torch.int64, device=DEV)
    out = torch.full((3, n, k), float("nan"), dtype=torch.bfloat16, device=DEV)
    plan = pkg.DeviceLensPlan(pkg.OP_WGRAD, pkg.DType.BF16, pkg.DType.BF16, 3, sum(gm), n, k, bad.data_ptr(), 0,
                              go.data_ptr(), x.data_ptr(), out.data_ptr(), _stream())
    plan.run(_stream())
    st, _, msg = plan.status(_stream())
    plan.release()
    assert st == pkg.GG_ERR_INVALID and "group 1" in msg, msg
    assert torch.count_nonzero(out[1].float()) == 0
    ref = go[:300].float().t().contiguous() @ x[:300].float()
    assert ((out[0].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
    # wrappers with device sizes
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    gw = pkg.grouped_gemm_wgrad(go, x, lens)
    ref = go[800:].float().t().contiguous() @ x[800:].float()
    assert ((gw[2].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
    w = _inputs(pkg, 0, 1, 3, n, k)[1]  # [3, n, k]
    gx = pkg.grouped_gemm_dgrad(go, w, lens)
    ref = go[300:800].float() @ w[1].float()
    assert ((gx[300:800].float() - ref).abs() <= ATOL + RTOL * ref.abs()).all()
    with pytest.raises(pkg.GGError):
        pkg.grouped_gemm_dgrad(go, w, torch.tensor([300, 500, 900], dtype=torch.int64, device=DEV))


# ---- the in-kernel table (at most 64 groups) and the table kernel (more) --------------------
@pytest.mark.parametrize("b", [64, 65, 130])
def test_table_paths_match_host_sizes(pkg, b):
    """Up to 64 groups the grouped GEMM builds the group table itself (one launch); above, a
    table kernel runs first. Both give the bits of the host-size plan, with ragged and empty
    groups, and report the tile count."""
    gen = torch.Generator().manual_seed(b)
    gm = torch.randint(0, 700, (b,), generator=gen).tolist()
    for g in range(0, b, 9):
        gm[g] = 0
    n, k = 520, 448
    x, w = _inputs(pkg, 0, sum(gm), b, n, k, seed_x=60 + b, seed_w=61 + b)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    print(f"[device-lens] {b} groups, {sum(gm)} rows: N={n} K={k}", flush=True)
    plan = DevicePlan(pkg, 0, x, w, lens)
    detail = plan.be.detail()
    assert ("in-kernel table" in detail) == (b <= 64), detail
    st, tiles, msg = plan.run()
    assert st == pkg.GG_OK, msg
    assert tiles == sum((m + 255) // 256 for m in gm) * ((n + 255) // 256), (tiles, detail)
    host = _host_plan_out(pkg, 0, x, w, gm)
    assert torch.equal(plan.out.view(torch.int16), host.view(torch.int16)), detail
    plan.close()


@pytest.mark.parametrize("b", [64, 65])
def test_table_paths_report_bad_sizes(pkg, b):
    """Both table paths name the first group whose rows do not fit, and compute the others."""
    gm = [40] * b
    gm[b - 3] = -1
    total = 40 * (b - 1)
    x, w = _inputs(pkg, 0, total, b, 264, 128, seed_x=70, seed_w=71)
    plan = DevicePlan(pkg, 0, x, w, torch.tensor(gm, dtype=torch.int64, device=DEV))
    st, _, msg = plan.run()
    assert st == pkg.GG_ERR_INVALID and f"group {b - 3}" in msg, msg
    _check_group(x, w, plan.out, 0, 0, 40)
    _check_group(x, w, plan.out, b - 1, 40 * (b - 2), 40)
    plan.close()


@pytest.mark.parametrize("kind", ["dgrad", "wgrad"])
def test_table_kernel_backward_matches_host_sizes(pkg, kind):
    """dgrad / wgrad with more than 64 groups (the table kernel path) give the host plan's bits."""
    gen = torch.Generator().manual_seed(80)
    gm = torch.randint(0, 300, (70,), generator=gen).tolist()
    gm[5] = 0
    n, k = 264, 392
    rows = sum(gm)
    go = torch.randn((rows, n), generator=gen).to(torch.bfloat16).to(DEV)
    other = torch.randn((len(gm), n, k) if kind == "dgrad" else (rows, k), generator=gen).to(torch.bfloat16).to(DEV)
    shape = (rows, k) if kind == "dgrad" else (len(gm), n, k)
    out = torch.full(shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    lens = torch.tensor(gm, dtype=torch.int64, device=DEV)
    plan = pkg.DeviceLensPlan(pkg.OP_DGRAD if kind == "dgrad" else pkg.OP_WGRAD, pkg.DType.BF16, pkg.DType.BF16,
                              len(gm), rows, n, k, lens.data_ptr(), 0, go.data_ptr(), other.data_ptr(),
                              out.data_ptr(), _stream(), 0, 0)
    plan.run(_stream())
    st, _, msg = plan.status(_stream())
    detail = plan.detail()
    plan.release()
    assert st == pkg.GG_OK, msg
    assert "in-kernel table" not in detail, detail
    host = _host_backward(pkg, kind, None, gm, n, k, go, other, None, None)
    assert torch.equal(out.view(torch.int16), host.view(torch.int16)), f"bits differ from host plan ({detail})"
