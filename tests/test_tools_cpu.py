"""The measurement tools' own logic, on the CPU: stamps.py (per-tile cycle budgets), trace.py
(kernel-trace summaries) and pmc.py (counter passes).

The figures in profiles/ come from these parsers, so each is checked against an independent
statement of what it reads:
- stamps.unchecked_steps against a literal run of the kernel's unchecked-loop bound
  (csrc/gg_kernel_impl.h: kt = 1, then kt += 6 while kt + 9 < T with tail masks, kt + 8 < T
  without);
- stamps.analyse against synthetic stamps with known segment lengths on per-workgroup clocks
  that are millions of cycles apart (shader clocks of different CUs are not synchronised);
- trace.mangled_instance / kernel_label against names written out by hand, and against the
  compiler's resource report of the built library when it is there;
- pmc.dispatches / mean_after_first / instance against a hand-written rocprofv3 CSV.
"""
import importlib.util
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "groupgemm-cktile-optimized_amd")


def _load(name):
    spec = importlib.util.spec_from_file_location(f"gg_tool_{name}", os.path.join(PKG_DIR, f"{name}.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


stamps = _load("stamps")
trace = _load("trace")
pmc = _load("pmc")


def _loop_steps(T, masks):
    lead = 9 if masks else 8
    kt, n = 1, 0
    while kt + lead < T:
        kt += 6
        n += 6
    return n


@pytest.mark.parametrize("masks", [False, True])
def test_unchecked_steps_follow_the_kernel_loop(masks):
    for T in range(1, 260):
        assert stamps.unchecked_steps(T, masks) == _loop_steps(T, masks), (T, masks)
    # the checked steps after the loop (K steps 1 + n .. T - 1): at most lead, and more than
    # lead - 6 whenever the loop ran
    lead = 9 if masks else 8
    for T in range(2, 260):
        n = stamps.unchecked_steps(T, masks)
        rest = T - 1 - n
        assert rest <= lead and (n == 0 or rest > lead - 6), (T, masks, rest)


def test_analyse_recovers_known_segments():
    T, masks = 45, False  # 36 unchecked steps
    per_step, first, lookup, checked, gap = 50, 100, 20, 540, 30
    prologue, epilogue = 500, 400
    tiles = [3, 1, 2, 7]
    st = np.zeros((len(tiles), 64), dtype=np.int64)
    for w, nt in enumerate(tiles):
        t = 10_000_000 * (w + 1) + 12_345 * w  # unrelated clocks per workgroup
        st[w, 0] = t
        t += prologue
        st[w, 1] = t
        for j in range(nt):
            s = 2 + 5 * j
            if j:
                t += gap
            st[w, s] = t
            t += first
            st[w, s + 1] = t
            t += 36 * per_step
            st[w, s + 2] = t
            t += lookup
            st[w, s + 3] = t
            t += checked
            st[w, s + 4] = t
        t += 10
        st[w, 62] = t
        st[w, 63] = t + epilogue
    r = stamps.analyse(st, T, masks)
    assert r["unchecked_steps_per_tile"] == 36
    assert r["tiles_per_wg_max"] == 7
    assert r["prologue"] == prologue and r["final_epilogue"] == epilogue
    assert r["first step"] == first and r["next tile lookup"] == lookup and r["checked"] == checked
    assert r["gap to next tile"] == gap
    assert r["unchecked_per_step"] == per_step
    tile = first + 36 * per_step + lookup + checked + gap
    assert r["tile_cycles"] == tile
    assert r["boundary"] == tile - T * per_step
    lens = [prologue + n * (first + 36 * per_step + lookup + checked) + (n - 1) * gap + 10 + epilogue
            for n in tiles]
    assert r["launch_cycles_mean"] == pytest.approx(np.mean(lens))
    assert r["launch_cycles_max"] == max(lens)


def test_analyse_without_unchecked_steps():
    st = np.zeros((2, 64), dtype=np.int64)
    for w in range(2):
        st[w, 0], st[w, 1] = 1000, 1100
        st[w, 2:7] = [1200, 1300, 1300, 1310, 1900]
        st[w, 62], st[w, 63] = 1950, 2300
    r = stamps.analyse(st, 8, True)
    assert r["unchecked_steps_per_tile"] == 0 and r["unchecked"] == 0
    assert np.isnan(r["unchecked_per_step"]) and "boundary" not in r
    assert r["gap to next tile"] == 0.0


def test_mangled_instance_and_label():
    name = "void gg::(anonymous namespace)::grouped_gemm_kernel<false, true, 13, 0, false, true>(gg::KernelArgs)"
    assert trace.mangled_instance(name) == "grouped_gemm_kernelILb0ELb1ELi13ELi0ELb0ELb1EE"
    assert trace.kernel_label(name) == "gg::grouped_gemm_kernel<false, true, 13, 0, false, true>"
    assert trace.kernel_label("gg::split_reduce_kernel<false, false>(float const*, int)") == \
        "gg::split_reduce_kernel<false, false>"
    assert trace.mangled_instance("gg::split_reduce_kernel<false, false>") == ""
    small = "void gg::(anonymous namespace)::small_gemm_kernel<true, false>(gg::SmallArgs)"
    assert trace.mangled_instance(small) == "small_gemm_kernelILb1ELb0EE"
    assert trace.kernel_label(small) == "gg::small_gemm_kernel<true, false>"
    assert pmc.instance(small) == "small_gemm_kernel<true, false>" and pmc.is_gemm(small)
    assert not pmc.is_gemm("gg::(anonymous namespace)::small_reduce_kernel<true>(gg::SmallArgs)")


def test_profiled_instances_are_in_the_resource_report():
    report = os.path.join(PKG_DIR, "lib", "resource_usage.txt")
    if not os.path.exists(report):
        pytest.skip("library not built")
    text = open(report).read()
    prof = os.path.join(ROOT, "profiles")
    names = set()
    for f in os.listdir(prof):
        if f.startswith("grouped_gemm_kernel_") and f.endswith(".md"):
            head = open(os.path.join(prof, f)).readline()
            if "`" in head:
                names.add(head.split("`")[1])
    assert names, "no kernel-trace summaries"
    for n in names:
        key = trace.mangled_instance(n)
        assert key and re.search(rf"_ZN2gg12_GLOBAL__N_1\d+{key}EvNS_\d+(KernelArgs|SmallArgs)E", text), n
        assert "not in the resource report" not in trace.resource_line(n), n


def test_pmc_csv_parsing(tmp_path):
    kname = "gg::grouped_gemm_kernel<false, true, 0, 0, false, false>(gg::KernelArgs)"
    cc = tmp_path / "x_counter_collection.csv"
    rows = ["Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value"]
    for d, v in [(3, 100.0), (7, 10.0), (9, 20.0)]:
        rows.append(f'{d},"{kname}",FETCH_SIZE,{v}')
    rows.append('5,"other_kernel",FETCH_SIZE,999')
    cc.write_text("\n".join(rows) + "\n")
    kt = tmp_path / "x_kernel_trace.csv"
    kt.write_text("Dispatch_Id,Kernel_Name,Start_Timestamp,End_Timestamp\n"
                  f'3,"{kname}",1000,3500\n')
    (tmp_path / "x_agent_info.csv").write_text("ignored\n")
    ds = pmc.dispatches([str(p) for p in tmp_path.iterdir()], lambda n: "grouped_gemm_kernel" in n)
    assert sorted(ds) == [3, 7, 9]
    assert ds[3]["ns"] == 2500 and ds[7]["ns"] is None
    assert pmc.mean_after_first(ds, "FETCH_SIZE") == 15.0  # the first dispatch is dropped
    assert pmc.mean_after_first({3: ds[3]}, "FETCH_SIZE") == 100.0
    assert pmc.mean_after_first(ds, "WRITE_SIZE") is None
    assert pmc.instance(kname) == "grouped_gemm_kernel<false, true, 0, 0, false, false>"


def test_probe_mhz_arithmetic():
    """Shader cycles over wall-clock seconds: 1.5e8 cycles in 1e7 ticks of a 100 MHz clock is
    0.1 s at 1500 MHz; no elapsed ticks is an error."""
    import __graft_entry__ as entry

    pkg = entry.load_package()
    assert abs(pkg.probe_mhz([10, 5, 10 + 150_000_000, 5 + 10_000_000, 100_000_000]) - 1500.0) < 1e-9
    with pytest.raises(ValueError):
        pkg.probe_mhz([1, 7, 2, 7, 100_000_000])
