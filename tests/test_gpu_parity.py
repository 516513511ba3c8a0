"""Parity of the gfx950 grouped GEMM (through the C ABI) with the CPU oracle.

Bar (bench/bench_main.cpp:235-271): every checked output within
|got - ref| <= 1e-2 + 1e-2 * |ref| of an fp32 reference on the same seeded N(0,1) inputs.
  * small problems (the plumbing config, tails, edge cases): every output vs the CPU oracle;
  * large configs: the reference driver's samples (4 corners + 256 random per group,
    mt19937_64(1234)) vs the CPU oracle, plus every output vs a torch fp32 matmul per group,
    plus a NaN-prefilled output (an unwritten tile fails);
  * exact cases: small-integer inputs whose fp32 sums are exact and representable give
    bit-exact 16-bit outputs; grouped and one-group-at-a-time launches agree bit for bit.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-2

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _tdtype(dt):
    return torch.bfloat16 if int(dt) == 0 else torch.float16


class Run:
    """One grouped GEMM through the C ABI: seeded inputs, NaN-prefilled output."""

    def __init__(self, pkg, dtype, group_m, n, k, seed_x=1, seed_w=2, x=None, w=None):
        self.pkg, self.dtype, self.group_m, self.n, self.k = pkg, dtype, list(group_m), n, k
        tot = sum(group_m)
        td = _tdtype(dtype)
        self.stream = torch.cuda.current_stream(DEV).cuda_stream
        if x is None:
            x = torch.empty((tot, k), dtype=td, device=DEV)
            pkg.fill_randn(dtype, x.data_ptr(), x.numel(), seed_x, self.stream)
        if w is None:
            w = torch.empty((len(group_m), n, k), dtype=td, device=DEV)
            pkg.fill_randn(dtype, w.data_ptr(), w.numel(), seed_w, self.stream)
        self.x, self.w = x, w
        self.out = torch.full((tot, n), float("nan"), dtype=td, device=DEV)

    def go(self):
        be = self.pkg.make_mi355x_backend()
        prob = self.pkg.GroupedGemmProblem(self.dtype, len(self.group_m), self.n, self.k, self.group_m,
                                           self.x.data_ptr(), self.w.data_ptr(), self.out.data_ptr())
        why = be.prepare(prob, self.stream)
        assert why == "", why
        be.run(self.stream)
        torch.cuda.synchronize(DEV)
        self.detail = be.detail()
        be.release()
        return self

    def oracle_full(self, oracle):
        ref = oracle.grouped_gemm(int(self.dtype), _bits(self.x), _bits(self.w), self.group_m)
        got = oracle.decode(int(self.dtype), _bits(self.out))
        return got, ref

    def check_full(self, oracle):
        got, ref = self.oracle_full(oracle)
        bad, mx = oracle.check(got, ref, ATOL, RTOL)
        assert bad == 0, f"{bad}/{got.size} outputs off, max abs err {mx} ({self.detail})"
        return mx

    def check_sampled(self, oracle):
        s = oracle.make_samples(len(self.group_m), self.n, self.group_m, 256)
        ref = oracle.sampled(int(self.dtype), _bits(self.x), _bits(self.w), s)
        rows = torch.from_numpy(s[:, 0]).to(DEV)
        cols = torch.from_numpy(s[:, 1]).to(DEV)
        got = self.out[rows, cols].float().cpu().numpy()
        bad, mx = oracle.check(got, ref, ATOL, RTOL)
        assert bad == 0, f"{bad}/{len(s)} samples off, max abs err {mx} ({self.detail})"
        return len(s), mx

    def check_torch_fp32(self):
        """Every output vs a torch fp32 matmul of the same inputs, group by group."""
        row = 0
        worst = 0.0
        for g, m in enumerate(self.group_m):
            if m == 0:
                continue
            ref = self.x[row:row + m].float() @ self.w[g].float().t().contiguous()
            got = self.out[row:row + m].float()
            assert not torch.isnan(got).any(), f"group {g}: unwritten (NaN) outputs"
            err = (got - ref).abs()
            lim = ATOL + RTOL * ref.abs()
            nbad = int((err > lim).sum())
            assert nbad == 0, f"group {g}: {nbad} outputs off, max err {float(err.max())}"
            worst = max(worst, float(err.max()))
            row += m
        return worst


CONFIGS = {
    # (dtype, B, M per group, N, K)
    "1_plumbing": (0, 4, 256, 512, 1024),
    "2_gate_up": (0, 8, 4096, 4096, 7168),
    "3_down": (0, 8, 4096, 7168, 2048),
    "4_dense_fp16": (1, 8, 4096, 14336, 4096),
    "4_dense_bf16": (0, 8, 4096, 14336, 4096),
    "5a_tails": (0, 32, 520, 2880, 2880),
    "5b_low_occupancy": (0, 1, 2048, 7168, 2048),
}


def test_config1_every_output(pkg, oracle):
    dt, b, m, n, k = CONFIGS["1_plumbing"]
    r = Run(pkg, pkg.DType(dt), [m] * b, n, k).go()
    r.check_full(oracle)


@pytest.mark.parametrize("name", [c for c in CONFIGS if c != "1_plumbing"])
def test_baseline_config(pkg, oracle, name):
    dt, b, m, n, k = CONFIGS[name]
    print(f"[parity] {name}: dtype={dt} B={b} M={m} N={n} K={k}", flush=True)
    r = Run(pkg, pkg.DType(dt), [m] * b, n, k).go()
    ns, mx = r.check_sampled(oracle)
    worst = r.check_torch_fp32()
    print(f"[parity] {name}: {ns} samples ok (max err {mx:.3g}), all outputs vs torch fp32 ok "
          f"(max err {worst:.3g}); {r.detail}", flush=True)


# Tails and edge cases: every output vs the oracle. (dtype, group_m, N, K)
EDGE = [
    (0, [300, 300, 300], 1024, 512),        # shapes/pad_test.csv 9002 (M tail)
    (0, [300, 300], 1000, 2048),            # 9003 (M and N tails)
    (0, [1024], 2880, 2880),                # 9004 (N tail, single group)
    (0, [1, 7, 255, 257], 264, 128),        # tiny and off-by-one M
    (0, [65, 0, 129, 0], 8, 64),            # empty groups in the middle and at the end, N = 8
    (1, [200, 56], 248, 72),                # fp16, K % 64 != 0
    (0, [96, 160], 520, 1000),              # K % 64 == 40
    (0, [33], 128, 8),                      # K = 8 (one partial K step)
    (1, [520, 520], 2880, 2880),            # 5a shape, fp16, 2 groups
    (0, [0, 0, 512], 512, 256),             # leading empty groups
    (0, [3000, 17, 900], 776, 136),         # unbalanced groups
]


@pytest.mark.parametrize("case", range(len(EDGE)))
def test_edge_every_output(pkg, oracle, case):
    dt, gm, n, k = EDGE[case]
    print(f"[parity] edge {case}: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    r = Run(pkg, pkg.DType(dt), gm, n, k).go()
    r.check_full(oracle)


@pytest.mark.parametrize("dt,k", [(0, 128), (1, 128), (0, 72), (1, 200)])
def test_exact_small_integers(pkg, oracle, dt, k):
    """Inputs in {-1, 0, 1}: every fp32 partial sum is an integer of magnitude <= K <= 256,
    exact in fp32 and in the 16-bit output, so the output must match bit for bit."""
    gen = torch.Generator().manual_seed(7 + k + dt)
    group_m, n = [130, 256, 3], 264
    td = _tdtype(dt)
    x = torch.randint(-1, 2, (sum(group_m), k), generator=gen).to(td).to(DEV)
    w = torch.randint(-1, 2, (len(group_m), n, k), generator=gen).to(td).to(DEV)
    r = Run(pkg, pkg.DType(dt), group_m, n, k, x=x, w=w).go()
    got, ref = r.oracle_full(oracle)
    want = oracle.encode(dt, ref)
    assert np.array_equal(_bits(r.out), want.reshape(r.out.shape)), "not bit-exact"


def test_grouped_equals_per_group(pkg, monkeypatch):
    """Each output's K accumulation order is independent of the grouping: launching all
    groups at once and one group at a time gives identical bits. (Split-K is off: the two
    launches would choose different K ranges, and so different fp32 summation orders.)"""
    monkeypatch.setenv("GG_SPLIT_K", "1")
    gm, n, k = [700, 256, 513 - 1], 1040, 1216
    r = Run(pkg, pkg.DType.BF16, gm, n, k).go()
    row = 0
    for g, m in enumerate(gm):
        one = Run(pkg, pkg.DType.BF16, [m], n, k, x=r.x[row:row + m].contiguous(),
                  w=r.w[g:g + 1].contiguous()).go()
        assert torch.equal(one.out.view(torch.int16), r.out[row:row + m].view(torch.int16)), g
        row += m


def test_k_zero_writes_zeros(pkg):
    r = Run(pkg, pkg.DType.BF16, [17, 5], 64, 0)
    r.go()
    assert torch.count_nonzero(r.out.float()) == 0


def test_repeated_runs_identical(pkg):
    """run() is re-entrant: back-to-back launches on one plan give the same bits."""
    dt, b, m, n, k = CONFIGS["5a_tails"]
    r = Run(pkg, pkg.DType(dt), [m] * 4, n, k)
    be = pkg.make_mi355x_backend()
    prob = pkg.GroupedGemmProblem(pkg.DType(dt), 4, n, k, [m] * 4, r.x.data_ptr(), r.w.data_ptr(),
                                  r.out.data_ptr())
    assert be.prepare(prob, r.stream) == ""
    be.run(r.stream)
    torch.cuda.synchronize(DEV)
    first = r.out.clone()
    for _ in range(5):
        be.run(r.stream)
    torch.cuda.synchronize(DEV)
    be.release()
    assert torch.equal(first.view(torch.int16), r.out.view(torch.int16))


def test_device_fill_matches_oracle_generator(pkg, oracle):
    """The device N(0,1) generator agrees with the host restatement to within one 16-bit ulp
    (device logf/cospif vs host log/cos), and is bit-identical for nearly every element."""
    for dt in (0, 1):
        cnt = 1 << 20
        t = torch.empty(cnt, dtype=_tdtype(dt), device=DEV)
        pkg.fill_randn(pkg.DType(dt), t.data_ptr(), cnt, 1, torch.cuda.current_stream(DEV).cuda_stream)
        torch.cuda.synchronize(DEV)
        dev_bits = _bits(t)
        host_bits = oracle.fill_randn(dt, cnt, 1)
        dv = oracle.decode(dt, dev_bits).astype(np.float64)
        hv = oracle.decode(dt, host_bits).astype(np.float64)
        # one 16-bit ulp is at most 2^-7 relative (bf16); tiny values may differ absolutely
        assert (np.abs(dv - hv) <= 2.0 ** -7 * np.abs(hv) + 1e-6).all()
        assert (dev_bits == host_bits).mean() > 0.99


@pytest.mark.parametrize("steps", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 13, 14, 16, 20, 31, 32, 33, 34, 35])
def test_k_step_counts_with_several_tiles_per_workgroup(pkg, steps):
    """Every K-step count mod 6 (the unrolled loop and its tail) and mod 2 / mod 3 (the LDS
    stage rotation between consecutive tiles of a workgroup), with 2 to 3 tiles per workgroup,
    every output against torch fp32. 1-3 steps take the per-tile variant, whose workgroups then
    run a prologue and an LDS epilogue per tile."""
    k = 64 * steps - (8 if steps % 4 == 1 else 0)  # some partial last steps too
    gm, n = [4096, 256], 8192
    print(f"[parity] K steps {steps}: K={k} group_m={gm} N={n}", flush=True)
    r = Run(pkg, pkg.DType.BF16, gm, n, k).go()
    r.check_torch_fp32()


# Multi-tile workgroups (cross-tile kernel): the previous tile's outputs are written from
# registers inside the next tile's first step. N % 256 == 8 leaves an 8-column last tile
# column, K % 64 != 0 a partial last step; some workgroups get two or three tiles.
CROSS_TAILS = [
    (0, [5000, 3100, 33], 2056, 1000),
    (1, [4100, 4100], 2568, 704),   # exactly 11 K steps, fp16
    (0, [2000, 9, 2047, 0, 1500], 4104, 2056),
]


@pytest.mark.parametrize("case", range(len(CROSS_TAILS)))
def test_register_epilogue_tails(pkg, oracle, case):
    dt, gm, n, k = CROSS_TAILS[case]
    print(f"[parity] register-epilogue tails {case}: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    r = Run(pkg, pkg.DType(dt), gm, n, k).go()
    assert "cross-tile" in r.detail, r.detail
    r.check_sampled(oracle)
    r.check_torch_fp32()

