"""The plug-in boundary and the drivers, without a GPU.

* mi355x_backend.cpp compiles unchanged against the reference's own common/backend.hpp
  (common/backend.hpp:63-83): the reference's driver needs one factory line to run it
  (bench/bench_main.cpp:398-407). Skipped where the reference tree is absent.
* The comparison library loads and exports its C shim; its stream-K rule reads Tensile kernel
  names the way the 4-stream loop's gate needs.
* gg_bench and the reference-driver build reject bad command lines before touching the device.
"""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "groupgemm-cktile-optimized_amd")
REF = "/root/reference"
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "common", "backend.hpp")), reason="no reference tree")
def test_backend_compiles_against_the_reference_header(tmp_path):
    # a copy in a directory without this repository's backend.hpp, so that #include "backend.hpp"
    # resolves to the reference's through -I
    src = tmp_path / "mi355x_backend.cpp"
    shutil.copy(os.path.join(PKG, "csrc", "host", "mi355x_backend.cpp"), src)
    r = subprocess.run([HIPCC, "-fsyntax-only", "-std=c++17", "-x", "hip", f"-I{REF}/common",
                        f"-I{ROOT}/include", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # the header it compiled against is the reference's (its factories, not this repository's registry)
    r = subprocess.run([HIPCC, "-E", "-std=c++17", "-x", "hip", f"-I{REF}/common", f"-I{ROOT}/include", str(src)],
                       capture_output=True, text=True)
    assert "make_ck_tile_backend" in r.stdout and "backend_registry" not in r.stdout


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "bench", "bench_main.cpp")), reason="no reference tree")
def test_reference_driver_builds_with_this_backend():
    exe = os.path.join(ROOT, "oracle", "_ref", "tunemax_bench")
    assert os.path.exists(exe), "oracle/_ref/tunemax_bench is built by __graft_entry__.build()"
    syms = subprocess.run(["nm", "-C", exe], capture_output=True, text=True).stdout
    # the driver's ck_tile factory resolves to this repository's backend
    assert re.search(r"\bT tunemax::make_mi355x_backend\(\)", syms)
    assert "make_ck_tile_backend" not in syms
    r = subprocess.run([exe, "--help"], capture_output=True, text=True)
    assert r.returncode == 2 and "--shapes" in r.stderr


def _cmp():
    import __graft_entry__ as entry

    return entry.load_package().load_compare_library()


def test_compare_library_exports_its_shim():
    lib = _cmp()
    for name in ("ggc_create", "ggc_prepare", "ggc_run", "ggc_release", "ggc_destroy", "ggc_message",
                 "ggc_detail", "ggc_heuristic_kernel", "ggc_is_stream_k"):
        assert hasattr(lib, name)
    assert lib.ggc_create(None, None) == 2
    assert lib.ggc_message(None) == b""


@pytest.mark.parametrize("name,sk", [
    ("Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_SK3_SNLL0_TLDS1_WG32_8_1", 1),
    ("Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_SK0_TLDS1", 0),
    ("Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_TLDS1", 0),
    ("Cijk_Alik_Bljk_SK1", 1),
    ("Cijk_Alik_Bljk_SKX_SK0_", 0),
    ("Cijk_ASK2_", 0),  # the token must start with an underscore: "_SK"
    ("", 0),
])
def test_stream_k_rule(name, sk):
    assert _cmp().ggc_is_stream_k(name.encode()) == sk


def test_gg_bench_rejects_bad_command_lines():
    exe = os.path.join(PKG, "bin", "gg_bench")
    r = subprocess.run([exe, "--bogus"], capture_output=True, text=True)
    assert r.returncode == 2 and "unknown argument --bogus" in r.stderr
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "--shapes is required" in r.stderr
    r = subprocess.run([exe, "--shapes", "x.csv", "--iters", "0"], capture_output=True, text=True)
    assert r.returncode == 2
    r = subprocess.run([exe, "--help"], capture_output=True, text=True)
    assert r.returncode == 0 and "--backends" in r.stdout
