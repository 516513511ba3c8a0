"""ctypes binding of the CPU oracle (oracle/lib/libgg_oracle.so) — TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product. See gg_oracle.h for what each function restates (reference file:line) and how it is
pinned.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "lib", "libgg_oracle.so")

_P16 = ctypes.POINTER(ctypes.c_uint16)
_PF = ctypes.POINTER(ctypes.c_float)
_PI64 = ctypes.POINTER(ctypes.c_int64)
_PU64 = ctypes.POINTER(ctypes.c_uint64)
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "gg_oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "gg_oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "gg_oracle_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "gg_oracle_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "gg_oracle_decode": (None, [ctypes.c_int, _P16, _PF, ctypes.c_size_t]),
            "gg_oracle_encode": (None, [ctypes.c_int, _PF, _P16, ctypes.c_size_t]),
            "gg_oracle_fp8_to_f32": (ctypes.c_float, [ctypes.c_int, ctypes.c_uint8]),
            "gg_oracle_grouped_gemm_fp8": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p]),
            "gg_oracle_grouped_dgrad_fp8": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                                   ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                                   ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                                   ctypes.c_void_p]),
            "gg_oracle_grouped_wgrad_fp8": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                                   ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                                   ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                                   ctypes.c_void_p]),
            "gg_oracle_grouped_dgrad": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p]),
            "gg_oracle_grouped_wgrad": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p]),
            "gg_oracle_grouped_gemm": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                              _PI64, _P16, _P16, _PF]),
            "gg_oracle_group_rows": (None, [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, _P16, _P16,
                                            ctypes.c_int64, _PF]),
            "gg_oracle_sampled": (None, [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, _P16, _P16, _PI64,
                                         ctypes.c_int64, _PF]),
            "gg_oracle_make_samples": (ctypes.c_int64, [ctypes.c_int, ctypes.c_int64, _PI64, ctypes.c_int,
                                                        _PI64]),
            "gg_oracle_check": (ctypes.c_int64, [_PF, _PF, ctypes.c_int64, ctypes.c_double, ctypes.c_double,
                                                 ctypes.POINTER(ctypes.c_double)]),
            "gg_oracle_fill_randn": (None, [ctypes.c_int, _P16, ctypes.c_size_t, ctypes.c_uint64]),
            "gg_oracle_splitmix64": (ctypes.c_uint64, [ctypes.c_uint64]),
            "gg_mt19937_64_seq": (None, [ctypes.c_uint64, _PU64, ctypes.c_size_t]),
            "gg_mt19937_64_nth": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
            "gg_oracle_threads": (ctypes.c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _ptr(a: np.ndarray, ct):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ct))


def decode(dtype: int, bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().gg_oracle_decode(dtype, _ptr(bits, ctypes.c_uint16), _ptr(out, ctypes.c_float), bits.size)
    return out


def encode(dtype: int, vals: np.ndarray) -> np.ndarray:
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.empty(vals.shape, dtype=np.uint16)
    lib().gg_oracle_encode(dtype, _ptr(vals, ctypes.c_float), _ptr(out, ctypes.c_uint16), vals.size)
    return out


def grouped_gemm(dtype: int, x: np.ndarray, w: np.ndarray, group_m) -> np.ndarray:
    """fp32 out [sum(M), N] from 16-bit bit patterns x [sum(M), K], w [B, N, K]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    b, n, k = w.shape
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    out = np.zeros((int(gm.sum()), n), dtype=np.float32)
    lib().gg_oracle_grouped_gemm(dtype, b, n, k, _ptr(gm, ctypes.c_int64), _ptr(x, ctypes.c_uint16),
                                 _ptr(w, ctypes.c_uint16), _ptr(out, ctypes.c_float))
    return out


def fp8_decode(fmt: int, b: np.ndarray) -> np.ndarray:
    """fp8 bytes (fmt 0: e4m3, 1: e5m2) -> fp32."""
    lut = np.array([lib().gg_oracle_fp8_to_f32(fmt, i) for i in range(256)], dtype=np.float32)
    return lut[np.asarray(b, dtype=np.uint8)]


def grouped_gemm_fp8(fmt: int, x: np.ndarray, w: np.ndarray, group_m, x_scale: float, w_scale) -> np.ndarray:
    """fp32 out [sum(M), N] = (x_g @ w_g^T) * x_scale * w_scale[g] from fp8 bytes x [sum(M), K],
    w [B, N, K]."""
    x = np.ascontiguousarray(x, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    b, n, k = w.shape
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    ws = np.ascontiguousarray(w_scale, dtype=np.float32)
    out = np.zeros((int(gm.sum()), n), dtype=np.float32)
    lib().gg_oracle_grouped_gemm_fp8(fmt, b, n, k, gm.ctypes.data, x.ctypes.data, w.ctypes.data, float(x_scale),
                                     ws.ctypes.data, out.ctypes.data)
    return out


def grouped_dgrad_fp8(a_fmt: int, b_fmt: int, grad_out: np.ndarray, w: np.ndarray, group_m, a_scale: float,
                      b_scale) -> np.ndarray:
    """fp32 grad_x [sum(M), K] = (grad_out [sum(M), N] @ w[g] [N, K]) * a_scale * b_scale[g] per
    group from fp8 bytes (formats 0: e4m3, 1: e5m2)."""
    grad_out = np.ascontiguousarray(grad_out, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    b, n, k = w.shape
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    bs = np.ascontiguousarray(b_scale, dtype=np.float32)
    out = np.zeros((int(gm.sum()), k), dtype=np.float32)
    lib().gg_oracle_grouped_dgrad_fp8(a_fmt, b_fmt, b, n, k, gm.ctypes.data, grad_out.ctypes.data, w.ctypes.data,
                                      float(a_scale), bs.ctypes.data, out.ctypes.data)
    return out


def grouped_wgrad_fp8(a_fmt: int, b_fmt: int, grad_out: np.ndarray, x: np.ndarray, group_m, a_scale: float,
                      b_scale) -> np.ndarray:
    """fp32 grad_w [B, N, K] = (grad_out[g]^T @ x[g]) * a_scale * b_scale[g] per group from fp8
    bytes; zero for an empty group."""
    grad_out = np.ascontiguousarray(grad_out, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.uint8)
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    bs = np.ascontiguousarray(b_scale, dtype=np.float32)
    n, k = grad_out.shape[1], x.shape[1]
    out = np.zeros((len(gm), n, k), dtype=np.float32)
    lib().gg_oracle_grouped_wgrad_fp8(a_fmt, b_fmt, len(gm), n, k, gm.ctypes.data, grad_out.ctypes.data,
                                      x.ctypes.data, float(a_scale), bs.ctypes.data, out.ctypes.data)
    return out


def grouped_dgrad(dtype: int, grad_out: np.ndarray, w: np.ndarray, group_m) -> np.ndarray:
    """fp32 grad_x [sum(M), K] = grad_out [sum(M), N] @ w[g] [N, K] per group (bit patterns in)."""
    grad_out = np.ascontiguousarray(grad_out, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    b, n, k = w.shape
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    out = np.zeros((int(gm.sum()), k), dtype=np.float32)
    lib().gg_oracle_grouped_dgrad(dtype, b, n, k, gm.ctypes.data, grad_out.ctypes.data, w.ctypes.data,
                                  out.ctypes.data)
    return out


def grouped_wgrad(dtype: int, grad_out: np.ndarray, x: np.ndarray, group_m) -> np.ndarray:
    """fp32 grad_w [B, N, K] = grad_out[g]^T [N, M_g] @ x[g] [M_g, K] per group; zero if M_g = 0."""
    grad_out = np.ascontiguousarray(grad_out, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    n, k = grad_out.shape[1], x.shape[1]
    out = np.zeros((len(gm), n, k), dtype=np.float32)
    lib().gg_oracle_grouped_wgrad(dtype, len(gm), n, k, gm.ctypes.data, grad_out.ctypes.data, x.ctypes.data,
                                  out.ctypes.data)
    return out


def group_rows(dtype: int, x_rows: np.ndarray, w_group: np.ndarray) -> np.ndarray:
    x_rows = np.ascontiguousarray(x_rows, dtype=np.uint16)
    w_group = np.ascontiguousarray(w_group, dtype=np.uint16)
    rows, k = x_rows.shape
    n = w_group.shape[0]
    out = np.empty((rows, n), dtype=np.float32)
    lib().gg_oracle_group_rows(dtype, n, k, _ptr(x_rows, ctypes.c_uint16), _ptr(w_group, ctypes.c_uint16),
                               rows, _ptr(out, ctypes.c_float))
    return out


def make_samples(group_num: int, n: int, group_m, per_group: int = 256) -> np.ndarray:
    gm = np.ascontiguousarray(group_m, dtype=np.int64)
    cnt = lib().gg_oracle_make_samples(group_num, n, _ptr(gm, ctypes.c_int64), per_group, None)
    out = np.empty((cnt, 3), dtype=np.int64)
    lib().gg_oracle_make_samples(group_num, n, _ptr(gm, ctypes.c_int64), per_group, _ptr(out, ctypes.c_int64))
    return out


def sampled(dtype: int, x: np.ndarray, w: np.ndarray, samples: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    samples = np.ascontiguousarray(samples, dtype=np.int64)
    _, n, k = w.shape
    ref = np.empty(samples.shape[0], dtype=np.float32)
    lib().gg_oracle_sampled(dtype, n, k, _ptr(x, ctypes.c_uint16), _ptr(w, ctypes.c_uint16),
                            _ptr(samples, ctypes.c_int64), samples.shape[0], _ptr(ref, ctypes.c_float))
    return ref


def check(got: np.ndarray, ref: np.ndarray, atol: float = 1e-2, rtol: float = 1e-2):
    """(mismatches, max_abs) under |got - ref| <= atol + rtol * |ref| (NaN -> mismatch, inf)."""
    got = np.ascontiguousarray(got, dtype=np.float32).ravel()
    ref = np.ascontiguousarray(ref, dtype=np.float32).ravel()
    assert got.size == ref.size
    mx = ctypes.c_double()
    bad = lib().gg_oracle_check(_ptr(got, ctypes.c_float), _ptr(ref, ctypes.c_float), got.size, atol, rtol,
                                ctypes.byref(mx))
    return int(bad), float(mx.value)


def fill_randn(dtype: int, count: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16)
    lib().gg_oracle_fill_randn(dtype, _ptr(out, ctypes.c_uint16), count, seed)
    return out


def splitmix64(z: int) -> int:
    """The input generator's splitmix64 stage: the next output of a splitmix64 in state z."""
    return int(lib().gg_oracle_splitmix64(z))


def mt19937_64(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint64)
    lib().gg_mt19937_64_seq(seed, _ptr(out, ctypes.c_uint64), count)
    return out


def mt19937_64_nth(seed: int, z: int) -> int:
    return int(lib().gg_mt19937_64_nth(seed, z))


def threads() -> int:
    return int(lib().gg_oracle_threads())
