"""Python host side of the MI355X grouped GEMM, over the C ABI in include/gg_grouped_gemm.h.

Mirrors the reference's backend interface (common/backend.hpp:39-83) so Python callers and
the tests read like the reference's driver (bench/bench_main.cpp:392-538):

  GroupedGemmProblem   common/backend.hpp:39-60   (dtype, group_num, n, k, group_m, x, w, out)
  Backend              common/backend.hpp:69-79   (name / prepare / run / release / detail)
  make_mi355x_backend  one more factory beside make_ck_tile_backend & co. (backend.hpp:81-83)

Device buffers are passed as raw device addresses (ints), e.g. ``tensor.data_ptr()``;
streams as raw hipStream_t handles (``torch.cuda.current_stream().cuda_stream``) or 0.
The compute path is the native library only: if ``lib/libgg_mi355x.so`` is missing, loading
raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libgg_mi355x.so")

GG_OK, GG_ERR_UNSUPPORTED, GG_ERR_INVALID, GG_ERR_HIP = 0, 1, 2, 3

# Every symbol include/gg_grouped_gemm.h declares, with its ctypes signature.
C_API = {
    "gg_prepare": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "gg_run": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "gg_release": (None, [ctypes.c_void_p]),
    "gg_plan_detail": (ctypes.c_char_p, [ctypes.c_void_p]),
    "gg_plan_grid": (ctypes.c_int, [ctypes.c_void_p]),
    "gg_plan_tiles": (ctypes.c_int, [ctypes.c_void_p]),
    "gg_last_error": (ctypes.c_char_p, []),
    "gg_fill_randn": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64,
                                     ctypes.c_void_p]),
}

_lib: Optional[ctypes.CDLL] = None


class GGError(RuntimeError):
    """A C ABI call failed; ``status`` is the gg_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"gg status {status}: {message}")
        self.status = status


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the native library (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"native grouped GEMM library missing: {path} (build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` at the repo root)")
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in C_API.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def last_error() -> str:
    return load_library().gg_last_error().decode()


def _check(status: int) -> None:
    if status != GG_OK:
        raise GGError(status, last_error())


class DType(enum.IntEnum):
    """tunemax::DType (common/backend.hpp:27)."""
    BF16 = 0
    FP16 = 1


def dtype_name(t: DType) -> str:
    return "bf16" if t == DType.BF16 else "fp16"


@dataclass
class GroupedGemmProblem:
    """Field-for-field the reference's GroupedGemmProblem (common/backend.hpp:39-60).

    x [sum(group_m), k], w [group_num, n, k], out [sum(group_m), n], all row-major device
    buffers given by address; out[rows of group g] = x[rows of group g] @ w[g]^T.
    """
    dtype: DType = DType.BF16
    group_num: int = 0
    n: int = 0
    k: int = 0
    group_m: List[int] = field(default_factory=list)
    x: int = 0
    w: int = 0
    out: int = 0
    group_lens_pinned: int = 0  # host address of the same lengths (unused by this backend)

    def total_m(self) -> int:
        return sum(self.group_m)

    def flops(self) -> float:
        return 2.0 * float(self.total_m()) * float(self.n) * float(self.k)


class Backend:
    """One grouped GEMM implementation (common/backend.hpp:63-79).

    prepare(): untimed; returns "" when ready, else the reason it cannot run (N/A).
    run():     timed; enqueues exactly one grouped GEMM on `stream`, no synchronization.
    release(): frees what prepare() allocated.
    """

    def name(self) -> str:
        raise NotImplementedError

    def prepare(self, problem: GroupedGemmProblem, stream: int = 0) -> str:
        raise NotImplementedError

    def run(self, stream: int = 0) -> None:
        raise NotImplementedError

    def release(self) -> None:
        pass

    def detail(self) -> str:
        return ""


class Mi355xBackend(Backend):
    """The hand-written gfx950 persistent grouped GEMM (libgg_mi355x.so)."""

    def __init__(self) -> None:
        self._lib = load_library()
        self._plan = ctypes.c_void_p()

    def name(self) -> str:
        return "mi355x"

    def prepare(self, problem: GroupedGemmProblem, stream: int = 0) -> str:
        self.release()
        gm = (ctypes.c_int64 * max(1, problem.group_num))(*problem.group_m)
        st = self._lib.gg_prepare(int(problem.dtype), problem.group_num, problem.n, problem.k, gm,
                                  problem.x, problem.w, problem.out, stream, ctypes.byref(self._plan))
        if st == GG_ERR_UNSUPPORTED:
            return last_error()
        _check(st)
        return ""

    def run(self, stream: int = 0) -> None:
        _check(self._lib.gg_run(self._plan, stream))

    def release(self) -> None:
        if self._plan:
            self._lib.gg_release(self._plan)
            self._plan = ctypes.c_void_p()

    def detail(self) -> str:
        return self._lib.gg_plan_detail(self._plan).decode() if self._plan else ""

    def grid(self) -> int:
        return self._lib.gg_plan_grid(self._plan) if self._plan else 0

    def tiles(self) -> int:
        return self._lib.gg_plan_tiles(self._plan) if self._plan else 0

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass


def make_mi355x_backend() -> Backend:
    return Mi355xBackend()


# Name -> factory registry (the reference hard-codes an if-chain, bench/bench_main.cpp:398-407).
BACKENDS = {"mi355x": make_mi355x_backend}


def make_backend(name: str) -> Backend:
    if name not in BACKENDS:
        raise KeyError(f"unknown backend {name!r}; known: {sorted(BACKENDS)}")
    return BACKENDS[name]()


def fill_randn(dtype: DType, ptr: int, count: int, seed: int, stream: int = 0) -> None:
    """Seeded N(0,1) device fill of the benchmark driver (bench/bench_main.cpp:160-176)."""
    _check(load_library().gg_fill_randn(int(dtype), ptr, count, seed, stream))


def grouped_gemm(x, w, group_m: Sequence[int], out=None, stream: Optional[int] = None):
    """out = grouped GEMM of torch tensors x [sum(M), K], w [B, N, K] (bf16 or fp16, cuda).

    Convenience wrapper: prepare + run + release on the current stream.
    """
    import torch

    if x.dtype != w.dtype or x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("x and w must both be bfloat16 or both float16")
    if not (x.is_cuda and w.is_cuda and x.is_contiguous() and w.is_contiguous()):
        raise ValueError("x and w must be contiguous device tensors")
    b, n, k = w.shape
    if len(group_m) != b or x.shape[1] != k or x.shape[0] != sum(group_m):
        raise ValueError("shape mismatch between x, w and group_m")
    if out is None:
        out = torch.empty((x.shape[0], n), dtype=x.dtype, device=x.device)
    s = torch.cuda.current_stream(x.device).cuda_stream if stream is None else stream
    prob = GroupedGemmProblem(DType.BF16 if x.dtype == torch.bfloat16 else DType.FP16, b, n, k,
                              list(group_m), x.data_ptr(), w.data_ptr(), out.data_ptr())
    be = Mi355xBackend()
    why = be.prepare(prob, s)
    if why:
        raise GGError(GG_ERR_UNSUPPORTED, why)
    try:
        be.run(s)
        # the plan's device table must outlive the launch
        torch.cuda.current_stream(x.device).synchronize()
    finally:
        be.release()
    return out
