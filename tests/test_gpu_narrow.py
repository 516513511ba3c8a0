"""Narrow tiles (256 x 224) for one-round forward problems, on the GPU.

A 16-bit forward plan whose 256-wide tiles fit in one round with CUs to spare, and which is not
split, takes tiles of 256 x 224 when those still fit in one round (1 x 2048 x 7168: 224 tiles of
256 x 256, 256 of 256 x 224). Every output is the same sequence of MFMAs over K whichever tile
holds it, so a narrow plan must give the bits of the 256-wide plan (GG_NARROW=0), and every output
within rtol = atol = 1e-2 of float32 (bench/bench_main.cpp:264-268). Outputs are NaN-prefilled.
Cases: the config 5b shape; ragged groups with M tails and a 208-column last tile; fp16 with a
104-column last tile (the second wave of that tile has no valid column).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

DEV = torch.device("cuda:0")
ATOL = RTOL = 1e-2

CASES = [
    (torch.bfloat16, [2048], 7168, 2048),          # config 5b: 224 -> 256 tiles
    (torch.bfloat16, [1000, 24, 513], 2000, 1088),  # 64 -> 72 tiles, M tails, last tile 208 columns
    (torch.float16, [300, 700, 129], 1000, 520),    # 20 -> 25 tiles, last tile 104 columns, K % 64 = 8
]


def _run(pkg, x, w, gm, narrow, monkeypatch):
    if narrow:
        monkeypatch.delenv("GG_NARROW", raising=False)
    else:
        monkeypatch.setenv("GG_NARROW", "0")
    b, n, k = w.shape
    out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device=DEV)
    s = torch.cuda.current_stream(DEV).cuda_stream
    be = pkg.make_mi355x_backend()
    dt = pkg.DType.BF16 if x.dtype == torch.bfloat16 else pkg.DType.FP16
    why = be.prepare(pkg.GroupedGemmProblem(dt, b, n, k, gm, x.data_ptr(), w.data_ptr(), out.data_ptr()), s)
    assert why == "", why
    be.run(s)
    torch.cuda.synchronize(DEV)
    detail = be.detail()
    be.release()
    return out, detail


@pytest.mark.parametrize("case", range(len(CASES)))
def test_narrow_tiles_match_wide(pkg, monkeypatch, case):
    dt, gm, n, k = CASES[case]
    print(f"[narrow] case {case}: dtype={dt} group_m={gm} N={n} K={k}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(90 + case)
    x = torch.randn((sum(gm), k), generator=g, device=DEV).to(dt)
    w = torch.randn((len(gm), n, k), generator=g, device=DEV).to(dt)
    narrow, d_narrow = _run(pkg, x, w, gm, True, monkeypatch)
    wide, d_wide = _run(pkg, x, w, gm, False, monkeypatch)
    assert "256x224" in d_narrow and "per-tile" in d_narrow, d_narrow
    assert "256x256" in d_wide, d_wide
    assert torch.equal(narrow.view(torch.int16), wide.view(torch.int16)), (d_narrow, d_wide)
    row = 0
    for gi, m in enumerate(gm):
        ref = x[row:row + m].float() @ w[gi].float().t().contiguous()
        got = narrow[row:row + m].float()
        assert not torch.isnan(got).any(), f"group {gi}: unwritten outputs"
        bad = int(((got - ref).abs() > ATOL + RTOL * ref.abs()).sum())
        assert bad == 0, f"group {gi}: {bad} outputs off"
        row += m
