"""The C ABI library without a GPU: it loads, exports every symbol include/*.h declares, and
rejects bad arguments / unsupported shapes before touching the device (no compute calls)."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(gg_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_the_entry_points():
    syms = _declared_symbols()
    for s in ("gg_prepare", "gg_run", "gg_release", "gg_last_error", "gg_plan_detail"):
        assert s in syms, syms


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load_library()
    missing = [s for s in _declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and as dynamic symbols of the shared object itself
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (gg_\w+)$", out, flags=re.M))
    assert set(_declared_symbols()) <= exported
    assert set(pkg.C_API) == set(_declared_symbols())


def _prepare(lib, dtype=0, group_num=2, n=64, k=64, group_m=(5, 6), x=16, w=16, out=16):
    plan = ctypes.c_void_p()
    gm = (ctypes.c_int64 * max(1, len(group_m)))(*group_m) if group_m is not None else None
    st = lib.gg_prepare(dtype, group_num, n, k, gm, x, w, out, None, ctypes.byref(plan))
    return st, plan


@pytest.mark.parametrize("kwargs,status,msg", [
    (dict(dtype=7), 2, "dtype"),
    (dict(n=-8), 2, ">= 0"),
    (dict(group_m=None), 2, "group_m is null"),
    (dict(group_m=(5, -1)), 2, "group_m[1] < 0"),
    (dict(x=0), 2, "device pointers"),
    (dict(n=12), 1, "N must be a multiple of 8"),
    (dict(k=20), 1, "K must be a multiple of 8"),
    (dict(out=24), 1, "16-byte aligned"),
    (dict(k=1 << 22), 1, "at most"),
])
def test_prepare_rejects_without_touching_the_gpu(pkg, kwargs, status, msg):
    lib = pkg.load_library()
    st, plan = _prepare(lib, **kwargs)
    assert st == status
    assert msg in pkg.last_error()
    assert not plan.value


def test_null_plan_paths(pkg):
    lib = pkg.load_library()
    assert lib.gg_run(None, None) == pkg.GG_ERR_INVALID
    lib.gg_release(None)
    assert lib.gg_plan_detail(None) == b""
    assert lib.gg_plan_grid(None) == 0 and lib.gg_plan_tiles(None) == 0
    plan = ctypes.c_void_p()
    assert lib.gg_prepare(0, 0, 8, 8, None, None, None, None, None, None) == pkg.GG_ERR_INVALID
    assert lib.gg_fill_randn(3, None, 0, 1, None) == pkg.GG_ERR_INVALID
    del plan


def test_backend_interface_mirrors_reference(pkg):
    """Backend / GroupedGemmProblem mirror common/backend.hpp:39-79."""
    be = pkg.make_backend("mi355x")
    assert be.name() == "mi355x"
    for meth in ("name", "prepare", "run", "release", "detail"):
        assert callable(getattr(be, meth))
    p = pkg.GroupedGemmProblem(pkg.DType.BF16, 3, 4096, 7168, [1, 2, 3])
    assert p.total_m() == 6 and p.flops() == 2.0 * 6 * 4096 * 7168
    assert pkg.dtype_name(pkg.DType.FP16) == "fp16"
    # unsupported shapes come back as an N/A reason, like a non-empty prepare() result
    p = pkg.GroupedGemmProblem(pkg.DType.BF16, 1, 12, 64, [4], 16, 16, 16)
    assert "multiple of 8" in be.prepare(p, 0)
    with pytest.raises(KeyError):
        pkg.make_backend("ck_tile_does_not_exist")


def _prepare_dev(lib, dtype=0, group_num=2, total_m=11, n=64, k=64, lens=16, offs=None, x=16, w=16,
                 out=16):
    plan = ctypes.c_void_p()
    st = lib.gg_prepare_device_lens(dtype, group_num, total_m, n, k, lens, offs, x, w, out, None,
                                    ctypes.byref(plan))
    return st, plan


@pytest.mark.parametrize("kwargs,status,msg", [
    (dict(dtype=5), 2, "dtype"),
    (dict(total_m=-1), 2, "total_m"),
    (dict(group_num=-2), 2, ">= 0"),
    (dict(lens=None), 2, "group_lens is null"),
    (dict(w=0), 2, "device pointers"),
    (dict(n=20), 1, "N must be a multiple of 8"),
    (dict(k=12), 1, "K must be a multiple of 8"),
    (dict(x=8), 1, "16-byte aligned"),
    (dict(n=1 << 22), 1, "at most"),
])
def test_prepare_device_lens_rejects_without_touching_the_gpu(pkg, kwargs, status, msg):
    """Device-resident group sizes: the same argument and shape rules as gg_prepare, checked
    without reading the sizes (they are device memory)."""
    lib = pkg.load_library()
    st, plan = _prepare_dev(lib, **kwargs)
    assert st == status
    assert msg in pkg.last_error()
    assert not plan.value


def test_device_lens_plans_without_work_need_no_gpu(pkg):
    """K == 0 or an empty output: the plan is built on the host alone; its status is OK."""
    lib = pkg.load_library()
    for kw, note in ((dict(k=0), "K = 0"), (dict(total_m=0), "empty output"), (dict(group_num=0), "empty")):
        st, plan = _prepare_dev(lib, **kw)
        assert st == pkg.GG_OK, pkg.last_error()
        assert note in lib.gg_plan_detail(plan).decode()
        tiles = ctypes.c_int(-1)
        assert lib.gg_plan_device_status(plan, None, ctypes.byref(tiles)) == pkg.GG_OK
        assert tiles.value == 0
        lib.gg_release(plan)
    assert lib.gg_plan_device_status(None, None, None) == pkg.GG_ERR_INVALID
    assert lib.gg_prepare_device_lens(0, 1, 8, 8, 8, 16, None, 16, 16, 16, None, None) == pkg.GG_ERR_INVALID


def test_compute_group_offs_rejects_bad_arguments(pkg):
    lib = pkg.load_library()
    assert lib.gg_compute_group_offs(None, 16, -1, None) == pkg.GG_ERR_INVALID
    assert lib.gg_compute_group_offs(None, 16, 4, None) == pkg.GG_ERR_INVALID
    assert lib.gg_compute_group_offs(16, None, 4, None) == pkg.GG_ERR_INVALID
