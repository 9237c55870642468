"""ctypes bindings for ``oracle/build/libhcp_oracle.so`` (TEST INFRASTRUCTURE).

Builds the library with ``make -C oracle`` when it is missing.  See ``hcp_oracle.c``
for what each function restates and the reference lines it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "libhcp_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        L.oracle_draw_normals.argtypes = [ctypes.c_uint64, ctypes.c_int,
                                          ctypes.POINTER(i64), ctypes.POINTER(vp), ctypes.c_int]
        L.oracle_draw_normals.restype = None
        L.oracle_draw_uniforms.argtypes = [ctypes.c_uint64, i64, vp]
        L.oracle_draw_uniforms.restype = None
        L.oracle_paged_gather.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, i64,
                                          vp, vp, i64, i64]
        L.oracle_paged_gather.restype = ctypes.c_int
        L.oracle_paged_scatter.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, i64,
                                           vp, vp, i64, i64, ctypes.c_int]
        L.oracle_paged_scatter.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def draw_normals(seed: int, shapes, kind: str):
    """Draw tensors of ``shapes`` from one stream.  kind: "f64" | "fp32" | "bf16"."""
    code = {"f64": 0, "fp32": 1, "bf16": 2}[kind]
    dt = {"f64": np.float64, "fp32": np.float32, "bf16": np.uint16}[kind]
    outs = [np.empty(shp, dtype=dt) for shp in shapes]
    n = len(outs)
    counts = (ctypes.c_int64 * n)(*[o.size for o in outs])
    ptrs = (ctypes.c_void_p * n)(*[_ptr(o) for o in outs])
    lib().oracle_draw_normals(ctypes.c_uint64(seed), n, counts, ptrs, code)
    return outs


def draw_uniforms(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    lib().oracle_draw_uniforms(ctypes.c_uint64(seed), n, _ptr(out))
    return out


def paged_gather(pool: np.ndarray, table: np.ndarray, table_seq_offset: int, t0: int, t1: int,
                 out_k: np.ndarray | None = None, out_v: np.ndarray | None = None):
    """pool [2, nb, bs, hkv, d] (uint16 or float32) -> (k, v) [hkv, t1-t0, d]."""
    assert pool.ndim == 5 and pool.shape[0] == 2 and pool.flags.c_contiguous
    _, nb, bs, hkv, d = pool.shape
    L = t1 - t0
    if out_k is None:
        out_k = np.zeros((hkv, L, d), dtype=pool.dtype)
        out_v = np.zeros((hkv, L, d), dtype=pool.dtype)
    table = np.ascontiguousarray(table, dtype=np.int32)
    rc = lib().oracle_paged_gather(_ptr(pool), nb, bs, hkv, d, pool.itemsize, _ptr(table),
                                   table.size, table_seq_offset, t0, t1, _ptr(out_k),
                                   _ptr(out_v), out_k.strides[0] // pool.itemsize,
                                   out_k.strides[1] // pool.itemsize)
    if rc != 0:
        raise ValueError(f"oracle_paged_gather rc={rc}")
    return out_k, out_v


def paged_scatter(pool: np.ndarray, table: np.ndarray, table_seq_offset: int, t0: int, t1: int,
                  k: np.ndarray, v: np.ndarray, zero_tail: bool = True) -> None:
    """In-place inverse of :func:`paged_gather` (k, v are [hkv, t1-t0, d])."""
    _, nb, bs, hkv, d = pool.shape
    table = np.ascontiguousarray(table, dtype=np.int32)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    rc = lib().oracle_paged_scatter(_ptr(pool), nb, bs, hkv, d, pool.itemsize, _ptr(table),
                                    table.size, table_seq_offset, t0, t1, _ptr(k), _ptr(v),
                                    k.strides[0] // pool.itemsize, k.strides[1] // pool.itemsize,
                                    1 if zero_tail else 0)
    if rc != 0:
        raise ValueError(f"oracle_paged_scatter rc={rc}")
