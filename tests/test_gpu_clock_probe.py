"""The clock probe (gg_clock_probe) on the GPU: it waits the asked wall-clock time and reports a
shader clock within the MI355X's range, alone and beside a run of the grouped GEMM, whose outputs
stay those of the same launches without it."""
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X", allow_module_level=True)

import __graft_entry__ as entry  # noqa: E402

DEV = torch.device("cuda:0")
MASK = (1 << 64) - 1


def _words(t):
    return [int(v) & MASK for v in t.cpu().tolist()]


def test_probe_alone_waits_and_reads_a_plausible_clock():
    pkg = entry.load_package()
    words = torch.zeros(5, dtype=torch.int64, device=DEV)
    pkg.clock_probe(words.data_ptr(), 0.02, torch.cuda.current_stream(DEV).cuda_stream)
    torch.cuda.synchronize()
    c0, t0, c1, t1, hz = _words(words)
    assert hz >= 1_000_000
    assert (t1 - t0) / hz >= 0.02
    assert 100.0 < pkg.probe_mhz([c0, t0, c1, t1, hz]) < 3000.0


def test_probe_beside_the_gemm():
    pkg = entry.load_package()
    b, m, n, k = 8, 1024, 2048, 2048
    x = torch.randn((b * m, k), device=DEV).to(torch.bfloat16)
    w = torch.randn((b, n, k), device=DEV).to(torch.bfloat16)
    outs = []
    stream = torch.cuda.current_stream(DEV)
    for with_probe in (False, True):
        out = torch.zeros((b * m, n), dtype=torch.bfloat16, device=DEV)
        be = pkg.make_mi355x_backend()
        assert not be.prepare(pkg.GroupedGemmProblem(pkg.DType.BF16, b, n, k, [m] * b, x.data_ptr(), w.data_ptr(),
                                                     out.data_ptr()), stream.cuda_stream)
        words = torch.zeros(5, dtype=torch.int64, device=DEV)
        side = torch.cuda.Stream(device=DEV)
        torch.cuda.synchronize()
        if with_probe:
            pkg.clock_probe(words.data_ptr(), 0.01, side.cuda_stream)
        for _ in range(50):
            be.run(stream.cuda_stream)
        torch.cuda.synchronize()
        be.release()
        outs.append(out)
        if with_probe:
            assert 100.0 < pkg.probe_mhz(_words(words)) < 3000.0
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
