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
    "gg_clock_probe": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_double, ctypes.c_void_p]),
    "gg_prepare_device_lens": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "gg_plan_device_status": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.POINTER(ctypes.c_int)]),
    "gg_compute_group_offs": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                             ctypes.c_void_p]),
    "gg_prepare_fp8": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_void_p)]),
    "gg_prepare_dgrad": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "gg_prepare_wgrad": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "gg_prepare_device_lens_op": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "gg_run_device_lens_noalloc": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                  ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_void_p]),
    "gg_prepare_dgrad_fp8": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "gg_prepare_wgrad_fp8": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
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
    """tunemax::DType (common/backend.hpp:27), plus the fp8 input types of gg_prepare_fp8."""
    BF16 = 0
    FP16 = 1
    FP8_E4M3 = 2
    FP8_E5M2 = 3


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
    group_lens_pinned: int = 0  # host address of the same lengths in pinned memory (unused here)

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

    def prepare_device_lens(self, dtype: DType, group_num: int, total_m: int, n: int, k: int,
                            group_lens: int, group_offs: int, x: int, w: int, out: int,
                            stream: int = 0) -> str:
        """Plan over device-resident group sizes (the group_lens_ptr / group_offs_ptr contract
        of the reference's Primus-Turbo grouped GEMM, grouped_gemm.h:35-36): group_lens is the
        device address of int64[group_num], group_offs of int64[group_num + 1] or 0. Every
        run() re-reads them on the stream. Returns "" or the reason it cannot run (N/A)."""
        self.release()
        st = self._lib.gg_prepare_device_lens(int(dtype), group_num, total_m, n, k, group_lens,
                                              group_offs or None, x, w, out, stream,
                                              ctypes.byref(self._plan))
        if st == GG_ERR_UNSUPPORTED:
            return last_error()
        _check(st)
        return ""

    def device_status(self, stream: int = 0):
        """(status, tile count, message) of the last run's device-side size check; synchronizes
        `stream` for device-size plans."""
        tiles = ctypes.c_int(0)
        st = self._lib.gg_plan_device_status(self._plan, stream, ctypes.byref(tiles))
        return st, tiles.value, last_error() if st != GG_OK else ""

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


class BackwardPlan:
    """A dgrad or wgrad plan (gg_prepare_dgrad / gg_prepare_wgrad), run any number of times.

    kind "dgrad": out [sum(M), k] = grad_out [sum(M), n] @ w[g] [n, k] per group.
    kind "wgrad": out [B, n, k] = grad_out[g]^T [n, M_g] @ x[g] [M_g, k], zero for empty groups.
    Buffers are device addresses; prepare raises GGError (status 1 = not supported).
    fp8 (gg_prepare_dgrad_fp8 / gg_prepare_wgrad_fp8): dtype is grad_out's fp8 type, other_dtype
    the other operand's (default: the same), grad_scale [1] and other_scale [B] device float32
    addresses; out is bf16, scaled by grad_scale[0] * other_scale[g].
    """

    def __init__(self, kind: str, dtype: DType, n: int, k: int, group_m: Sequence[int], grad_out: int,
                 other: int, out: int, stream: int = 0, other_dtype: Optional[DType] = None,
                 grad_scale: int = 0, other_scale: int = 0) -> None:
        if kind not in ("dgrad", "wgrad"):
            raise ValueError("kind must be 'dgrad' or 'wgrad'")
        self._lib = load_library()
        self._plan = ctypes.c_void_p()
        gm = (ctypes.c_int64 * max(1, len(group_m)))(*group_m)
        if int(dtype) in (int(DType.FP8_E4M3), int(DType.FP8_E5M2)):
            od = dtype if other_dtype is None else other_dtype
            fn = self._lib.gg_prepare_dgrad_fp8 if kind == "dgrad" else self._lib.gg_prepare_wgrad_fp8
            _check(fn(int(dtype), int(od), len(group_m), n, k, gm, grad_out, other, grad_scale, other_scale, out,
                      stream, ctypes.byref(self._plan)))
        else:
            fn = self._lib.gg_prepare_dgrad if kind == "dgrad" else self._lib.gg_prepare_wgrad
            _check(fn(int(dtype), len(group_m), n, k, gm, grad_out, other, out, stream, ctypes.byref(self._plan)))
        self.kind = kind
        self.flop = 2.0 * float(sum(group_m)) * float(n) * float(k)

    def run(self, stream: int = 0) -> None:
        _check(self._lib.gg_run(self._plan, stream))

    def detail(self) -> str:
        return self._lib.gg_plan_detail(self._plan).decode() if self._plan else ""

    def release(self) -> None:
        if self._plan:
            self._lib.gg_release(self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass


OP_FORWARD, OP_DGRAD, OP_WGRAD = 0, 1, 2  # gg_op


class DeviceLensPlan:
    """A plan over device-resident group sizes for any pass (gg_prepare_device_lens_op): op
    OP_FORWARD / OP_DGRAD / OP_WGRAD, a_dtype / b_dtype the input types (fp8 with device float32
    scales a_scale [1], b_scale [group_num]). Every run re-reads group_lens (and group_offs, or 0
    for back-to-back groups) on the stream; status() reports sizes that did not fit."""

    def __init__(self, op: int, a_dtype: DType, b_dtype: DType, group_num: int, total_m: int, n: int, k: int,
                 group_lens: int, group_offs: int, a: int, b: int, out: int, stream: int = 0,
                 a_scale: int = 0, b_scale: int = 0) -> None:
        self._lib = load_library()
        self._plan = ctypes.c_void_p()
        _check(self._lib.gg_prepare_device_lens_op(op, int(a_dtype), int(b_dtype), group_num, total_m, n, k,
                                                   group_lens, group_offs or None, a, b, a_scale or None,
                                                   b_scale or None, out, stream, ctypes.byref(self._plan)))

    def run(self, stream: int = 0) -> None:
        _check(self._lib.gg_run(self._plan, stream))

    def status(self, stream: int = 0):
        """(status, tile count, message) of the last run's device-side size check; synchronizes."""
        tiles = ctypes.c_int(0)
        st = self._lib.gg_plan_device_status(self._plan, stream, ctypes.byref(tiles))
        return st, tiles.value, last_error() if st != GG_OK else ""

    def detail(self) -> str:
        return self._lib.gg_plan_detail(self._plan).decode() if self._plan else ""

    def release(self) -> None:
        if self._plan:
            self._lib.gg_release(self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass


def run_device_lens_noalloc(op: int, a_dtype: DType, b_dtype: DType, group_num: int, total_m: int, n: int,
                            k: int, group_lens: int, group_offs: int, a: int, b: int, out: int, stream: int = 0,
                            a_scale: int = 0, b_scale: int = 0) -> None:
    """gg_run_device_lens_noalloc: DeviceLensPlan(...).run(stream) in one call that allocates no
    device memory (the group table lives in the library's per-GPU scratch array; at most 8192
    groups; calls that overlap on one GPU race on it)."""
    lib = load_library()
    _check(lib.gg_run_device_lens_noalloc(op, int(a_dtype), int(b_dtype), group_num, total_m, n, k, group_lens,
                                          group_offs or None, a, b, a_scale or None, b_scale or None, out,
                                          stream))


def _device_sizes(group_m, group_offs, b):
    """Validates device group sizes (and offsets); True if group_m is a device tensor."""
    import torch

    if not isinstance(group_m, torch.Tensor):
        if group_offs is not None:
            raise ValueError("group_offs goes with device group sizes")
        return False
    if not (group_m.is_cuda and group_m.dtype == torch.int64 and group_m.numel() == b and group_m.is_contiguous()):
        raise ValueError("device group sizes must be a contiguous int64 cuda tensor of B entries")
    if group_offs is not None and not (group_offs.is_cuda and group_offs.dtype == torch.int64
                                       and group_offs.numel() == b + 1 and group_offs.is_contiguous()):
        raise ValueError("group_offs must be a contiguous int64 cuda tensor of B + 1 entries")
    return True


def _run_device_plan(plan: DeviceLensPlan, s: int, dev) -> None:
    import torch

    try:
        plan.run(s)
        st, _, msg = plan.status(s)
        if st != GG_OK:
            raise GGError(st, msg)
        torch.cuda.current_stream(dev).synchronize()
    finally:
        plan.release()


class Fp8Plan:
    """An fp8 forward plan (gg_prepare_fp8): out (bf16) = (x[g] @ w[g]^T) * x_scale[0] *
    w_scale[g], tensor-wise scales in device memory (float32). Run any number of times."""

    def __init__(self, dtype: DType, n: int, k: int, group_m: Sequence[int], x: int, w: int, x_scale: int,
                 w_scale: int, out: int, stream: int = 0) -> None:
        self._lib = load_library()
        self._plan = ctypes.c_void_p()
        gm = (ctypes.c_int64 * max(1, len(group_m)))(*group_m)
        _check(self._lib.gg_prepare_fp8(int(dtype), len(group_m), n, k, gm, x, w, x_scale, w_scale, out, stream,
                                        ctypes.byref(self._plan)))
        self.flop = 2.0 * float(sum(group_m)) * float(n) * float(k)

    def run(self, stream: int = 0) -> None:
        _check(self._lib.gg_run(self._plan, stream))

    def detail(self) -> str:
        return self._lib.gg_plan_detail(self._plan).decode() if self._plan else ""

    def release(self) -> None:
        if self._plan:
            self._lib.gg_release(self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass


def grouped_gemm_fp8(x, w, group_m: Sequence[int], x_scale, w_scale, out=None, stream: Optional[int] = None):
    """bf16 out = (x[g] @ w[g]^T) * x_scale * w_scale[g] for torch float8_e4m3fn or float8_e5m2
    tensors x [sum(M), K], w [B, N, K] and float32 device scales x_scale [1], w_scale [B]."""
    import torch

    kinds = {torch.float8_e4m3fn: DType.FP8_E4M3, torch.float8_e5m2: DType.FP8_E5M2}
    if x.dtype != w.dtype or x.dtype not in kinds:
        raise TypeError("x and w must both be float8_e4m3fn or both float8_e5m2")
    if not (x_scale.dtype == w_scale.dtype == torch.float32 and x_scale.is_cuda and w_scale.is_cuda):
        raise TypeError("scales must be float32 device tensors")
    b, n, k = w.shape
    if len(group_m) != b or x.shape[1] != k or x.shape[0] != sum(group_m) or w_scale.numel() != b:
        raise ValueError("shape mismatch between x, w, group_m and the scales")
    if out is None:
        out = torch.empty((x.shape[0], n), dtype=torch.bfloat16, device=x.device)
    s = torch.cuda.current_stream(x.device).cuda_stream if stream is None else stream
    plan = Fp8Plan(kinds[x.dtype], n, k, list(group_m), x.data_ptr(), w.data_ptr(), x_scale.data_ptr(),
                   w_scale.data_ptr(), out.data_ptr(), s)
    try:
        plan.run(s)
        torch.cuda.current_stream(x.device).synchronize()
    finally:
        plan.release()
    return out


def make_mi355x_backend() -> Backend:
    return Mi355xBackend()


COMPARE_LIB_PATH = os.path.join(PKG_DIR, "lib", "libgg_compare.so")
_cmp_lib: Optional[ctypes.CDLL] = None


def load_compare_library(path: str = COMPARE_LIB_PATH) -> ctypes.CDLL:
    """The hipBLASLt comparison library's C shim (csrc/host/gg_compare.h); baselines, not the
    product. Load it in a process that has not imported torch: torch ships its own libhipblaslt
    under the same soname, and once that is loaded the shim's hipBLASLt calls resolve to it
    instead of the ROCm library it was built against. Drivers time the comparators in the
    native gg_bench (bench.py runs it as a child process)."""
    global _cmp_lib
    if _cmp_lib is None:
        if not os.path.exists(path):
            raise OSError(f"{path} is missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(path)
        sig = {
            "ggc_create": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
            "ggc_prepare": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                           ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
            "ggc_run": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
            "ggc_release": (None, [ctypes.c_void_p]),
            "ggc_destroy": (None, [ctypes.c_void_p]),
            "ggc_message": (ctypes.c_char_p, [ctypes.c_void_p]),
            "ggc_detail": (ctypes.c_char_p, [ctypes.c_void_p]),
            "ggc_heuristic_kernel": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                                    ctypes.c_char_p, ctypes.c_size_t]),
            "ggc_is_stream_k": (ctypes.c_int, [ctypes.c_char_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _cmp_lib = lib
    return _cmp_lib


def heuristic_kernel(dtype: DType, n: int, m: int, k: int):
    """(is stream-K, kernel name) of hipBLASLt's first choice for one group's out^T [n x m] over
    depth k, from the heuristic alone (no launch)."""
    buf = ctypes.create_string_buffer(1024)
    st = load_compare_library().ggc_heuristic_kernel(int(dtype), n, m, k, buf, len(buf))
    if st < 0:
        raise GGError(GG_ERR_HIP, buf.value.decode())
    return st == 1, buf.value.decode()


# Name -> factory registry (the reference hard-codes an if-chain, bench/bench_main.cpp:398-407).
# The hipBLASLt comparators are in the native driver's registry (bin/gg_bench).
BACKENDS = {"mi355x": make_mi355x_backend}

# Sources that decide which kernel runs and what it does: a profile measured on one build is
# matched to the current one by their hash (kernel_source_sha).
KERNEL_SOURCES = ("csrc/gg_kernel_impl.h", "csrc/gg_schedule.h", "csrc/gg_kernel.h", "csrc/gg_inst.hip", "csrc/gg_small.hip",
                  "csrc/gg_kernel.hip", "csrc/gg_capi.hip")


def kernel_source_sha() -> str:
    """First 16 hex digits of the SHA-256 over KERNEL_SOURCES (name and bytes of each)."""
    import hashlib

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update(rel.encode() + b"\0")
        with open(os.path.join(PKG_DIR, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def make_backend(name: str) -> Backend:
    if name not in BACKENDS:
        raise KeyError(f"unknown backend {name!r}; known: {sorted(BACKENDS)}")
    return BACKENDS[name]()


def fill_randn(dtype: DType, ptr: int, count: int, seed: int, stream: int = 0) -> None:
    """Seeded N(0,1) device fill of the benchmark driver (bench/bench_main.cpp:160-176)."""
    _check(load_library().gg_fill_randn(int(dtype), ptr, count, seed, stream))


def clock_probe(dev_out: int, seconds: float, stream: int = 0) -> None:
    """Enqueue the clock probe (gg_clock_probe): after it ran, the five uint64 at dev_out are the
    shader clock counter and the wall clock at its start and end, and the wall clock's rate in Hz."""
    _check(load_library().gg_clock_probe(dev_out, float(seconds), stream))


def probe_mhz(words) -> float:
    """Effective shader clock (MHz) from the five words clock_probe wrote."""
    c0, t0, c1, t1, hz = (int(v) for v in words)
    if t1 <= t0 or hz <= 0:
        raise ValueError("clock probe: no wall-clock ticks elapsed")
    return (c1 - c0) / ((t1 - t0) / hz) / 1e6


def _backward_shapes(kind, grad_out, other, group_m, device_sizes):
    n = grad_out.shape[1]
    b = group_m.numel() if device_sizes else len(group_m)
    if not device_sizes and grad_out.shape[0] != sum(group_m):
        raise ValueError("grad_out must have sum(group_m) rows")
    if kind == "dgrad":
        if other.shape[0] != b or other.shape[1] != n:
            raise ValueError("w must be [B, N, K] with N = grad_out's columns")
        k = other.shape[2]
        return n, k, (grad_out.shape[0], k)
    if other.shape[0] != grad_out.shape[0]:
        raise ValueError("x must have the rows of grad_out")
    k = other.shape[1]
    return n, k, (b, n, k)


def _backward(kind: str, grad_out, other, group_m, out, stream: Optional[int], group_offs=None):
    import torch

    if grad_out.dtype != other.dtype or grad_out.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("operands must both be bfloat16 or both float16")
    if not (grad_out.is_cuda and other.is_cuda and grad_out.is_contiguous() and other.is_contiguous()):
        raise ValueError("operands must be contiguous device tensors")
    b = group_m.numel() if isinstance(group_m, torch.Tensor) else len(group_m)
    device_sizes = _device_sizes(group_m, group_offs, b)
    n, k, shape = _backward_shapes(kind, grad_out, other, group_m, device_sizes)
    if out is None:
        out = torch.empty(shape, dtype=grad_out.dtype, device=grad_out.device)
    s = torch.cuda.current_stream(grad_out.device).cuda_stream if stream is None else stream
    dt = DType.BF16 if grad_out.dtype == torch.bfloat16 else DType.FP16
    if device_sizes:
        plan = DeviceLensPlan(OP_DGRAD if kind == "dgrad" else OP_WGRAD, dt, dt, b, grad_out.shape[0], n, k,
                              group_m.data_ptr(), group_offs.data_ptr() if group_offs is not None else 0,
                              grad_out.data_ptr(), other.data_ptr(), out.data_ptr(), s)
        _run_device_plan(plan, s, grad_out.device)
        return out
    plan = BackwardPlan(kind, dt, n, k, list(group_m), grad_out.data_ptr(), other.data_ptr(), out.data_ptr(), s)
    try:
        plan.run(s)
        torch.cuda.current_stream(grad_out.device).synchronize()
    finally:
        plan.release()
    return out


def _backward_fp8(kind: str, grad_out, other, group_m, grad_scale, other_scale, out, stream, group_offs=None):
    import torch

    kinds = {torch.float8_e4m3fn: DType.FP8_E4M3, torch.float8_e5m2: DType.FP8_E5M2}
    if grad_out.dtype not in kinds or other.dtype not in kinds:
        raise TypeError("operands must be float8_e4m3fn or float8_e5m2")
    if not (grad_out.is_cuda and other.is_cuda and grad_out.is_contiguous() and other.is_contiguous()):
        raise ValueError("operands must be contiguous device tensors")
    if not (grad_scale.dtype == other_scale.dtype == torch.float32 and grad_scale.is_cuda and other_scale.is_cuda):
        raise TypeError("scales must be float32 device tensors")
    b = group_m.numel() if isinstance(group_m, torch.Tensor) else len(group_m)
    device_sizes = _device_sizes(group_m, group_offs, b)
    if other_scale.numel() != b:
        raise ValueError("other_scale must hold one value per group")
    n, k, shape = _backward_shapes(kind, grad_out, other, group_m, device_sizes)
    if out is None:
        out = torch.empty(shape, dtype=torch.bfloat16, device=grad_out.device)
    s = torch.cuda.current_stream(grad_out.device).cuda_stream if stream is None else stream
    if device_sizes:
        plan = DeviceLensPlan(OP_DGRAD if kind == "dgrad" else OP_WGRAD, kinds[grad_out.dtype], kinds[other.dtype],
                              b, grad_out.shape[0], n, k, group_m.data_ptr(),
                              group_offs.data_ptr() if group_offs is not None else 0, grad_out.data_ptr(),
                              other.data_ptr(), out.data_ptr(), s, grad_scale.data_ptr(), other_scale.data_ptr())
        _run_device_plan(plan, s, grad_out.device)
        return out
    plan = BackwardPlan(kind, kinds[grad_out.dtype], n, k, list(group_m), grad_out.data_ptr(), other.data_ptr(),
                        out.data_ptr(), s, other_dtype=kinds[other.dtype], grad_scale=grad_scale.data_ptr(),
                        other_scale=other_scale.data_ptr())
    try:
        plan.run(s)
        torch.cuda.current_stream(grad_out.device).synchronize()
    finally:
        plan.release()
    return out


def grouped_gemm_dgrad_fp8(grad_out, w, group_m, grad_scale, w_scale, out=None, stream: Optional[int] = None,
                           group_offs=None):
    """bf16 grad_x = (grad_out [sum(M), N] @ w[g] [N, K]) * grad_scale * w_scale[g] for float8
    tensors (gradient e4m3 or e5m2, w e4m3 or matching) and float32 device scales. group_m: host
    sequence, or device int64 tensor (with optional device offsets), as for grouped_gemm."""
    return _backward_fp8("dgrad", grad_out, w, group_m, grad_scale, w_scale, out, stream, group_offs)


def grouped_gemm_wgrad_fp8(grad_out, x, group_m, grad_scale, x_scale, out=None, stream: Optional[int] = None,
                           group_offs=None):
    """bf16 grad_w [B, N, K] = (grad_out[g]^T @ x[g]) * grad_scale * x_scale[g] for float8 tensors,
    zero for empty groups. group_m: host sequence or device int64 tensor."""
    return _backward_fp8("wgrad", grad_out, x, group_m, grad_scale, x_scale, out, stream, group_offs)


def grouped_gemm_dgrad(grad_out, w, group_m, out=None, stream: Optional[int] = None, group_offs=None):
    """grad_x [sum(M), K] = grad_out [sum(M), N] @ w[g] [N, K] per group (torch tensors). group_m:
    host sequence, or device int64 tensor (with optional device offsets), as for grouped_gemm."""
    return _backward("dgrad", grad_out, w, group_m, out, stream, group_offs)


def grouped_gemm_wgrad(grad_out, x, group_m, out=None, stream: Optional[int] = None, group_offs=None):
    """grad_w [B, N, K] = grad_out[g]^T @ x[g] per group, zero for empty groups (torch tensors).
    group_m: host sequence or device int64 tensor."""
    return _backward("wgrad", grad_out, x, group_m, out, stream, group_offs)


def compute_group_offs(group_lens, stream: Optional[int] = None):
    """Device int64 offsets [B + 1] of back-to-back groups from device int64 lengths [B]
    (primus_turbo::compute_group_offs, grouped_gemm.h:138-140), on the current stream."""
    import torch

    if not (group_lens.is_cuda and group_lens.dtype == torch.int64 and group_lens.is_contiguous()):
        raise ValueError("group_lens must be a contiguous int64 cuda tensor")
    offs = torch.empty(group_lens.numel() + 1, dtype=torch.int64, device=group_lens.device)
    s = torch.cuda.current_stream(group_lens.device).cuda_stream if stream is None else stream
    _check(load_library().gg_compute_group_offs(group_lens.data_ptr(), offs.data_ptr(),
                                                group_lens.numel(), s))
    return offs


def grouped_gemm(x, w, group_m, out=None, stream: Optional[int] = None, group_offs=None):
    """out = grouped GEMM of torch tensors x [sum(M), K], w [B, N, K] (bf16 or fp16, cuda).

    group_m is a host sequence of row counts, or a device int64 tensor [B] of them (routing
    output; never read on the host, with optional device int64 offsets `group_offs` [B + 1],
    as the reference's Primus-Turbo grouped GEMM takes them). With device sizes, rows of x and
    out outside every group are left alone, and a size that does not fit raises GGError after
    the run. Convenience wrapper: prepare + run + release on the current stream.
    """
    import torch

    if x.dtype != w.dtype or x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("x and w must both be bfloat16 or both float16")
    if not (x.is_cuda and w.is_cuda and x.is_contiguous() and w.is_contiguous()):
        raise ValueError("x and w must be contiguous device tensors")
    b, n, k = w.shape
    device_sizes = isinstance(group_m, torch.Tensor)
    if device_sizes:
        if not (group_m.is_cuda and group_m.dtype == torch.int64 and group_m.numel() == b
                and group_m.is_contiguous()):
            raise ValueError("device group sizes must be a contiguous int64 cuda tensor of B entries")
        if group_offs is not None and not (group_offs.is_cuda and group_offs.dtype == torch.int64
                                           and group_offs.numel() == b + 1 and group_offs.is_contiguous()):
            raise ValueError("group_offs must be a contiguous int64 cuda tensor of B + 1 entries")
        if x.shape[1] != k:
            raise ValueError("shape mismatch between x and w")
    elif len(group_m) != b or x.shape[1] != k or x.shape[0] != sum(group_m):
        raise ValueError("shape mismatch between x, w and group_m")
    if out is None:
        out = torch.empty((x.shape[0], n), dtype=x.dtype, device=x.device)
    s = torch.cuda.current_stream(x.device).cuda_stream if stream is None else stream
    dt = DType.BF16 if x.dtype == torch.bfloat16 else DType.FP16
    be = Mi355xBackend()
    if device_sizes:
        why = be.prepare_device_lens(dt, b, x.shape[0], n, k, group_m.data_ptr(),
                                     group_offs.data_ptr() if group_offs is not None else 0,
                                     x.data_ptr(), w.data_ptr(), out.data_ptr(), s)
    else:
        why = be.prepare(GroupedGemmProblem(dt, b, n, k, list(group_m), x.data_ptr(), w.data_ptr(),
                                            out.data_ptr()), s)
    if why:
        raise GGError(GG_ERR_UNSUPPORTED, why)
    try:
        be.run(s)
        if device_sizes:
            st, _, msg = be.device_status(s)
            if st != GG_OK:
                raise GGError(st, msg)
        # the plan's device table must outlive the launch
        torch.cuda.current_stream(x.device).synchronize()
    finally:
        be.release()
    return out
