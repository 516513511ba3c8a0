"""Pins the CPU oracle (oracle/gg_oracle.c) before anything is checked against it.

Each check is independent of the oracle's own formulas: the C++ standard's known answer and
libstdc++'s engine for mt19937_64, numpy/torch conversions for the 16-bit formats, numpy
float64 / int64 matmul for the GEMM, and the reference driver's specification
(bench/bench_main.cpp:208-271) for the sampler and the tolerance rule.
"""
import json
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


# --------------------------------------------------------------------------------------
# mt19937_64 (the sampler's engine)
# --------------------------------------------------------------------------------------
def test_mt19937_64_standard_known_answer(oracle):
    # C++ standard [rand.predef]: the 10000th output of a default-constructed mt19937_64
    assert oracle.mt19937_64_nth(5489, 10000) == 9981545732273789042


def test_mt19937_64_matches_libstdcxx(oracle):
    with open(os.path.join(HERE, "golden", "mt19937_64.json")) as f:
        gold = json.load(f)
    for seed in (1234, 5489):
        want = np.array([int(v) for v in gold[f"seed_{seed}"]], dtype=np.uint64)
        assert np.array_equal(oracle.mt19937_64(seed, len(want)), want)
    assert oracle.mt19937_64_nth(5489, 10000) == int(gold["default_10000th"])


# --------------------------------------------------------------------------------------
# 16-bit formats
# --------------------------------------------------------------------------------------
def test_bf16_decode_all_patterns(oracle):
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = oracle.decode(0, bits)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp16_decode_all_patterns(oracle):
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = oracle.decode(1, bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _encode_cases():
    rng = np.random.default_rng(3)
    v = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 50,
        rng.standard_normal(20000).astype(np.float32) * 1e-5,           # fp16 subnormals
        (rng.integers(0, 1 << 16, 40000) << 16 | 0x8000).astype(np.uint32).view(np.float32),  # bf16 ties
        (rng.integers(0, 1 << 16, 40000) << 16 | 0x7fff).astype(np.uint32).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 65536, 3e38, -3e38,
                  6.1035156e-05, 6.0e-08, 2.98e-08, 2.99e-08, 1.0009765625, 1.00048828125],
                 dtype=np.float32),
    ])
    return v[np.isfinite(v) | np.isinf(v)]


def test_bf16_encode_rne(oracle):
    v = _encode_cases()
    got = oracle.encode(0, v)
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_fp16_encode_rne(oracle):
    v = _encode_cases()
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    got = oracle.encode(1, v)
    assert np.array_equal(got, want)


def test_encode_nan_stays_nan(oracle):
    v = np.array([np.nan, -np.nan], dtype=np.float32)
    for dt in (0, 1):
        assert np.isnan(oracle.decode(dt, oracle.encode(dt, v))).all()


# --------------------------------------------------------------------------------------
# the grouped GEMM
# --------------------------------------------------------------------------------------
def _rand_problem(dt, group_m, n, k, seed):
    rng = np.random.default_rng(seed)
    tot = sum(group_m)
    x = oracle_encode_np(dt, rng.standard_normal((tot, k)).astype(np.float32))
    w = oracle_encode_np(dt, rng.standard_normal((len(group_m), n, k)).astype(np.float32))
    return x, w


def oracle_encode_np(dt, v):
    if dt == 0:
        return torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return v.astype(np.float16).view(np.uint16)


def _decode_np(dt, b):
    if dt == 0:
        return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy()
    return b.view(np.float16).astype(np.float32)


@pytest.mark.parametrize("dt,group_m,n,k", [
    (0, [5, 0, 17, 1], 24, 40),
    (1, [33, 2], 8, 7),
    (0, [0, 0], 16, 16),
    (0, [64, 64, 64], 72, 129),
    (1, [300], 40, 1000),
])
def test_grouped_gemm_vs_numpy_float64(oracle, dt, group_m, n, k):
    """Per group out_g = x_g @ w_g^T (numpy float64 on the same decoded inputs)."""
    x, w = _rand_problem(dt, group_m, n, k, seed=k + n)
    got = oracle.grouped_gemm(dt, x, w, group_m)
    xf, wf = _decode_np(dt, x).astype(np.float64), _decode_np(dt, w).astype(np.float64)
    row = 0
    for g, m in enumerate(group_m):
        want = xf[row:row + m] @ wf[g].T
        np.testing.assert_allclose(got[row:row + m], want, rtol=1e-4, atol=1e-4 * np.sqrt(k))
        row += m
    assert got.shape == (sum(group_m), n)


def test_grouped_gemm_exact_integers(oracle):
    """Small integers: every fp32 partial sum is exact, so the result equals int64 matmul."""
    rng = np.random.default_rng(11)
    group_m, n, k = [7, 0, 12, 30], 20, 77
    xi = rng.integers(-8, 9, (sum(group_m), k))
    wi = rng.integers(-8, 9, (len(group_m), n, k))
    x = oracle_encode_np(0, xi.astype(np.float32))
    w = oracle_encode_np(0, wi.astype(np.float32))
    got = oracle.grouped_gemm(0, x, w, group_m)
    row = 0
    for g, m in enumerate(group_m):
        assert np.array_equal(got[row:row + m].astype(np.int64), xi[row:row + m] @ wi[g].T)
        row += m


@pytest.mark.parametrize("dt,group_m,n,k", [
    (0, [5, 0, 17, 1], 24, 40),
    (1, [33, 2], 8, 72),
    (0, [0, 0], 16, 16),
    (0, [64, 64, 64], 72, 129),
])
def test_grouped_dgrad_vs_numpy_float64(oracle, dt, group_m, n, k):
    """grad_x_g = grad_out_g @ w_g (w_g used as stored, N x K: a transposed w would fail)."""
    rng = np.random.default_rng(n * 7 + k)
    go = oracle_encode_np(dt, rng.standard_normal((sum(group_m), n)).astype(np.float32))
    w = oracle_encode_np(dt, rng.standard_normal((len(group_m), n, k)).astype(np.float32))
    got = oracle.grouped_dgrad(dt, go, w, group_m)
    gof, wf = _decode_np(dt, go).astype(np.float64), _decode_np(dt, w).astype(np.float64)
    assert got.shape == (sum(group_m), k)
    row = 0
    for g, m in enumerate(group_m):
        np.testing.assert_allclose(got[row:row + m], gof[row:row + m] @ wf[g], rtol=1e-4,
                                   atol=1e-4 * np.sqrt(n))
        row += m


@pytest.mark.parametrize("dt,group_m,n,k", [
    (0, [5, 0, 17, 1], 24, 40),
    (1, [33, 2], 8, 72),
    (0, [0, 0], 16, 16),
    (0, [64, 3, 100], 72, 129),
])
def test_grouped_wgrad_vs_numpy_float64(oracle, dt, group_m, n, k):
    """grad_w_g = grad_out_g^T @ x_g over the group's own rows; zero for an empty group."""
    rng = np.random.default_rng(n * 5 + k)
    go = oracle_encode_np(dt, rng.standard_normal((sum(group_m), n)).astype(np.float32))
    x = oracle_encode_np(dt, rng.standard_normal((sum(group_m), k)).astype(np.float32))
    got = oracle.grouped_wgrad(dt, go, x, group_m)
    gof, xf = _decode_np(dt, go).astype(np.float64), _decode_np(dt, x).astype(np.float64)
    assert got.shape == (len(group_m), n, k)
    row = 0
    for g, m in enumerate(group_m):
        want = gof[row:row + m].T @ xf[row:row + m] if m else np.zeros((n, k))
        np.testing.assert_allclose(got[g], want, rtol=1e-4, atol=1e-4 * np.sqrt(max(m, 1)))
        row += m


def test_backward_exact_integers(oracle):
    """Small integers: every fp32 partial sum is exact, so dgrad and wgrad equal int64 matmuls;
    dgrad of the forward's own w and wgrad agree with the forward by the product rule
    sum(grad_out * (x @ w^T)) = sum(grad_w * w) = sum(grad_x * x)."""
    rng = np.random.default_rng(5)
    group_m, n, k = [9, 0, 14, 3], 24, 40
    gi = rng.integers(-4, 5, (sum(group_m), n))
    xi = rng.integers(-4, 5, (sum(group_m), k))
    wi = rng.integers(-4, 5, (len(group_m), n, k))
    enc = lambda a: oracle_encode_np(0, a.astype(np.float32))
    gx = oracle.grouped_dgrad(0, enc(gi), enc(wi), group_m).astype(np.int64)
    gw = oracle.grouped_wgrad(0, enc(gi), enc(xi), group_m).astype(np.int64)
    out = oracle.grouped_gemm(0, enc(xi), enc(wi), group_m).astype(np.int64)
    row = 0
    for g, m in enumerate(group_m):
        assert np.array_equal(gx[row:row + m], gi[row:row + m] @ wi[g])
        assert np.array_equal(gw[g], gi[row:row + m].T @ xi[row:row + m])
        row += m
    assert (gi * out).sum() == (gw * wi).sum() == (gx * xi).sum()


@pytest.mark.parametrize("fmt,tdt", [(0, torch.float8_e4m3fn), (1, torch.float8_e5m2)])
def test_fp8_decode_all_patterns(oracle, fmt, tdt):
    """Every fp8 byte against torch's OCP float8 types (NaN patterns included)."""
    b = np.arange(256, dtype=np.uint8)
    got = oracle.fp8_decode(fmt, b)
    want = torch.from_numpy(b).view(tdt).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


@pytest.mark.parametrize("fmt", [0, 1])
def test_grouped_gemm_fp8_vs_numpy_float64(oracle, fmt):
    """fp8 GEMM with tensor-wise scales vs numpy float64 on the decoded inputs."""
    rng = np.random.default_rng(3 + fmt)
    group_m, n, k = [5, 0, 40, 17], 24, 160
    tdt = torch.float8_e4m3fn if fmt == 0 else torch.float8_e5m2
    x = torch.from_numpy(rng.standard_normal((sum(group_m), k)).astype(np.float32)).to(tdt).view(torch.uint8).numpy()
    w = torch.from_numpy(rng.standard_normal((len(group_m), n, k)).astype(np.float32)).to(tdt).view(torch.uint8).numpy()
    ws = np.array([0.5, 2.0, 0.25, 3.0], dtype=np.float32)
    got = oracle.grouped_gemm_fp8(fmt, x, w, group_m, 1.5, ws)
    xf, wf = oracle.fp8_decode(fmt, x).astype(np.float64), oracle.fp8_decode(fmt, w).astype(np.float64)
    row = 0
    for g, m in enumerate(group_m):
        want = (xf[row:row + m] @ wf[g].T) * 1.5 * ws[g]
        np.testing.assert_allclose(got[row:row + m], want, rtol=1e-4, atol=1e-4 * np.sqrt(k))
        row += m


@pytest.mark.parametrize("a_fmt,b_fmt", [(0, 0), (1, 1), (1, 0)])
def test_backward_fp8_vs_numpy_float64(oracle, a_fmt, b_fmt):
    """fp8 dgrad and wgrad (per-operand formats, tensor-wise gradient scale, per-group scale of
    the other operand) vs numpy float64 on the decoded inputs; an empty group's wgrad is 0."""
    rng = np.random.default_rng(11 + 2 * a_fmt + b_fmt)
    tdt = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}
    q = lambda shape, fmt: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(tdt[fmt]) \
        .view(torch.uint8).numpy()
    group_m, n, k = [7, 0, 33, 12], 48, 40
    go = q((sum(group_m), n), a_fmt)
    w = q((len(group_m), n, k), b_fmt)
    x = q((sum(group_m), k), b_fmt)
    bs = np.array([0.5, 4.0, 0.25, 2.0], dtype=np.float32)
    gx = oracle.grouped_dgrad_fp8(a_fmt, b_fmt, go, w, group_m, 1.5, bs)
    gw = oracle.grouped_wgrad_fp8(a_fmt, b_fmt, go, x, group_m, 1.5, bs)
    gof = oracle.fp8_decode(a_fmt, go).astype(np.float64)
    wf, xf = oracle.fp8_decode(b_fmt, w).astype(np.float64), oracle.fp8_decode(b_fmt, x).astype(np.float64)
    row = 0
    for g, m in enumerate(group_m):
        np.testing.assert_allclose(gx[row:row + m], gof[row:row + m] @ wf[g] * 1.5 * bs[g], rtol=1e-4,
                                   atol=1e-4 * np.sqrt(n))
        want = gof[row:row + m].T @ xf[row:row + m] * 1.5 * bs[g] if m else np.zeros((n, k))
        np.testing.assert_allclose(gw[g], want, rtol=1e-4, atol=1e-4 * np.sqrt(max(m, 1)))
        row += m


def test_backward_fp8_product_rule_and_mixed_formats(oracle):
    """Small integers in e4m3 and e5m2 (both exact): the fp8 dgrad / wgrad equal int64 matmuls,
    the 16-bit oracle's results on the same values, and satisfy the product rule with the fp8
    forward. A swapped operand or format fails these."""
    rng = np.random.default_rng(7)
    group_m, n, k = [9, 0, 14, 3], 32, 48
    gi = rng.integers(-3, 4, (sum(group_m), n))
    xi = rng.integers(-3, 4, (sum(group_m), k))
    wi = rng.integers(-3, 4, (len(group_m), n, k))
    f8 = lambda a, fmt: torch.from_numpy(a.astype(np.float32)).to(
        torch.float8_e5m2 if fmt else torch.float8_e4m3fn).view(torch.uint8).numpy()
    ones = np.ones(len(group_m), dtype=np.float32)
    gx = oracle.grouped_dgrad_fp8(1, 0, f8(gi, 1), f8(wi, 0), group_m, 1.0, ones).astype(np.int64)
    gw = oracle.grouped_wgrad_fp8(1, 0, f8(gi, 1), f8(xi, 0), group_m, 1.0, ones).astype(np.int64)
    out = oracle.grouped_gemm_fp8(0, f8(xi, 0), f8(wi, 0), group_m, 1.0, ones).astype(np.int64)
    enc = lambda a: oracle_encode_np(0, a.astype(np.float32))
    assert np.array_equal(gx, oracle.grouped_dgrad(0, enc(gi), enc(wi), group_m).astype(np.int64))
    assert np.array_equal(gw, oracle.grouped_wgrad(0, enc(gi), enc(xi), group_m).astype(np.int64))
    row = 0
    for g, m in enumerate(group_m):
        assert np.array_equal(gx[row:row + m], gi[row:row + m] @ wi[g])
        assert np.array_equal(gw[g], gi[row:row + m].T @ xi[row:row + m])
        row += m
    assert (gi * out).sum() == (gw * wi).sum() == (gx * xi).sum()


def test_group_rows_and_sampled_agree_with_full(oracle):
    dt, group_m, n, k = 0, [40, 9, 33], 56, 200
    x, w = _rand_problem(dt, group_m, n, k, seed=5)
    full = oracle.grouped_gemm(dt, x, w, group_m)
    part = oracle.group_rows(dt, x[40:49], w[1])
    np.testing.assert_allclose(part, full[40:49], rtol=1e-6, atol=1e-5)
    s = oracle.make_samples(len(group_m), n, group_m, 256)
    ref = oracle.sampled(dt, x, w, s)
    np.testing.assert_allclose(ref, full[s[:, 0], s[:, 1]], rtol=1e-5, atol=1e-4)


# --------------------------------------------------------------------------------------
# sampler (bench/bench_main.cpp:208-227)
# --------------------------------------------------------------------------------------
def test_samples_follow_reference_rule(oracle):
    group_m, n = [5, 0, 300, 1], 1000
    s = oracle.make_samples(len(group_m), n, group_m, 256)
    assert s.shape == (3 * 260, 3)  # empty groups get none
    seq = oracle.mt19937_64(1234, 2 * 256 * 3)  # one engine for all groups, row draw first
    pos, draw, row0 = 0, 0, 0
    for g, m in enumerate(group_m):
        if m == 0:
            continue
        corners = [(row0, 0), (row0, n - 1), (row0 + m - 1, 0), (row0 + m - 1, n - 1)]
        assert [tuple(r[:2]) for r in s[pos:pos + 4]] == corners
        for i in range(256):
            r, c, gg = s[pos + 4 + i]
            assert gg == g and row0 <= r < row0 + m and 0 <= c < n
            assert r == row0 + int(seq[draw]) % m and c == int(seq[draw + 1]) % n
            draw += 2
        pos += 260
        row0 += m


# --------------------------------------------------------------------------------------
# tolerance rule (bench/bench_main.cpp:235-271)
# --------------------------------------------------------------------------------------
def test_check_rule(oracle):
    ref = np.array([0.0, 100.0, -100.0, 5.0, 1.0, 1.0], dtype=np.float32)
    got = np.array([0.01, 101.0, -101.5, 5.0, np.nan, np.inf], dtype=np.float32)
    bad, mx = oracle.check(got, ref)
    # 0.01 <= 0.01 pass; 1.0 <= 1.01 pass; 1.5 > 1.01 fail; exact pass; NaN fail; inf fail
    assert bad == 3
    assert mx == np.inf
    bad, mx = oracle.check(got[:4], ref[:4])
    assert bad == 1 and abs(mx - 1.5) < 1e-6


# --------------------------------------------------------------------------------------
# input generator (bench/bench_main.cpp:160-176); exact bits unpinned (device math library)
# --------------------------------------------------------------------------------------
# splitmix64 (Steele, Lea and Flood 2014; Vigna's splitmix64.c): the published first outputs of
# the generator seeded with 0, which are also java.util.SplittableRandom(0)'s first nextLong()
# values. The stage is stateless in the fill (state = seed ^ index * 0x2545F4914F6CDD1D), so the
# n-th output is splitmix64(n * 0x9E3779B97F4A7C15). A wrong constant, shift or order fails this.
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC,
                    0x1B39896A51A8749B]


def test_splitmix64_known_answers(oracle):
    gamma = 0x9E3779B97F4A7C15
    for i, want in enumerate(SPLITMIX64_SEED0):
        assert oracle.splitmix64((i * gamma) % (1 << 64)) == want, i


def test_fill_uses_splitmix_of_seed_xor_scaled_index(oracle):
    """Element i of the fill is a function of splitmix64(seed ^ i * 0x2545F4914F6CDD1D) alone: two
    (seed, index) pairs with the same splitmix input give the same element (bench_main.cpp:170)."""
    c = 0x2545F4914F6CDD1D
    mask = (1 << 64) - 1
    i, j, seed_i = 3, 17, 1
    seed_j = seed_i ^ ((i * c) & mask) ^ ((j * c) & mask)
    a = oracle.fill_randn(0, i + 1, seed_i)[i]
    b = oracle.fill_randn(0, j + 1, seed_j)[j]
    assert a == b
@pytest.mark.parametrize("dt", [0, 1])
def test_fill_randn_is_standard_normal(oracle, dt):
    from scipy import stats

    v = _decode_np(dt, oracle.fill_randn(dt, 400000, 1)).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert stats.kstest(v, "norm").statistic < 0.01
    assert np.array_equal(oracle.fill_randn(dt, 1000, 1), oracle.fill_randn(dt, 4000, 1)[:1000])
    assert not np.array_equal(oracle.fill_randn(dt, 1000, 1), oracle.fill_randn(dt, 1000, 2))


# Closed forms of the Box-Muller stage (bench_main.cpp:171-173). With r the splitmix64 output:
# a 24-bit u2 field ((r >> 16) & 0xFFFFFF) of 0 gives cos(0) = 1, so the value is
# +sqrt(-2 ln u1); a u2 field of 0x800000 gives cos(pi) = -1, so -sqrt(-2 ln u1); r >> 40 ==
# 0xFFFFFF gives u1 = 1 exactly (the float 1/16777217 rounds to 2^-24), so a signed zero.
# u1 = ((r >> 40) + 1) * 2^-24 is exact in float. The indices were found by scanning the fill's
# splitmix64 inputs (seed ^ i * 0x2545F4914F6CDD1D) once; each case's condition is re-derived
# here through the pinned splitmix64 stage. Swapped bit fields, sin for cos, a lost sign or
# (r >> 40) without the + 1 each fail one of them.
BOX_MULLER_CASES = [(1, 10663227, "cos_one"), (2, 14069789, "cos_minus_one"), (2, 1888246, "u1_one")]


@pytest.mark.parametrize("dt", [0, 1])
def test_fill_box_muller_closed_forms(oracle, dt):
    c, mask = 0x2545F4914F6CDD1D, (1 << 64) - 1
    for seed, i, case in BOX_MULLER_CASES:
        r = oracle.splitmix64(seed ^ ((i * c) & mask))
        u2_field, hi = (r >> 16) & 0xFFFFFF, r >> 40
        u1 = (hi + 1) / float(1 << 24)
        got = int(oracle.fill_randn(dt, i + 1, seed)[i])
        if case == "u1_one":
            assert hi == 0xFFFFFF
            assert got & 0x7FFF == 0, hex(got)  # +0 or -0
            continue
        assert u2_field == (0 if case == "cos_one" else 0x800000)
        v = np.float32((1.0 if case == "cos_one" else -1.0) * np.sqrt(-2.0 * np.log(u1)))
        if dt == 0:
            want = int(torch.tensor([v]).to(torch.bfloat16).view(torch.int16).item()) & 0xFFFF
        else:
            want = int(np.array([v]).astype(np.float16).view(np.uint16)[0])
        assert got == want, (case, hex(got), hex(want), float(v))
