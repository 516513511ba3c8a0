"""The results comparison tool (groupgemm-cktile-optimized_amd/compare.py) on hand-made CSVs:
wins, geomean speedup and the pairing rules of the reference's scripts/compare.py:1-28."""
import csv
import importlib.util
import math
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
spec = importlib.util.spec_from_file_location(
    "gg_compare", os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "compare.py"))
cmp = importlib.util.module_from_spec(spec)
spec.loader.exec_module(cmp)

FIELDS = ["TestID", "Case", "B", "M", "N", "K", "Dtype", "GPU", "Backend", "Check", "Time_ms", "TFLOPS",
          "MaxAbsErr", "Detail"]


def _row(i, backend, ms, check="PASS"):
    flop = 1e9
    return dict(TestID=i, Case=f"c{i}", B=1, M=256, N=256, K=64, Dtype="bf16", GPU="x", Backend=backend,
                Check=check, Time_ms=ms, TFLOPS=flop / (ms * 1e-3) / 1e12, MaxAbsErr=0, Detail="")


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        w.writerows(rows)


def test_backend_comparison(tmp_path):
    rows = [_row(1, "mi355x", 1.0), _row(1, "hipblaslt_loop", 2.0),
            _row(2, "mi355x", 3.0), _row(2, "hipblaslt_loop", 1.5),
            _row(3, "mi355x", 1.0, "FAIL"), _row(3, "hipblaslt_loop", 1.0),
            _row(4, "mi355x", 1.0), _row(4, "hipblaslt_loop", 1.0, "N/A")]
    _write(tmp_path / "r.csv", rows)
    out = cmp.compare_backends(cmp.read_rows([str(tmp_path)]), "mi355x", "hipblaslt_loop")
    assert out[0].startswith("2 cases where both pass; mi355x faster in 1/2")
    assert "[3]" in out[0]  # the failing case is listed, the N/A one is not
    geo = math.sqrt((2.0 / 1.0) * (1.5 / 3.0))
    assert f"{geo:.3f}x" in out[1] and "4.000 ms vs 3.500 ms" in out[1]
    assert out[4].strip().startswith("2 ")  # worst case first: case 2 (0.5x)


def test_run_comparison(tmp_path):
    _write(tmp_path / "old.csv", [_row(1, "mi355x", 2.0), _row(2, "mi355x", 2.0)])
    _write(tmp_path / "new.csv", [_row(1, "mi355x", 1.0), _row(2, "mi355x", 2.5)])
    out = cmp.compare_runs(cmp.read_rows([str(tmp_path / "old.csv")]), cmp.read_rows([str(tmp_path / "new.csv")]),
                           "mi355x")
    assert out[0].startswith("2 cases where both pass; new mi355x faster in 1/2")
    assert f"{math.sqrt(2.0 * 0.8):.3f}x" in out[1]


def test_cli_needs_inputs(tmp_path, capsys):
    _write(tmp_path / "r.csv", [_row(1, "mi355x", 1.0), _row(1, "hipblaslt_loop", 2.0)])
    assert cmp.main([str(tmp_path / "r.csv")]) == 0
    assert "mi355x faster in 1/1" in capsys.readouterr().out
