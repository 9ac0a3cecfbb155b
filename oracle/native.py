"""ctypes binding of oracle/cpu_native.c (built by oracle/Makefile into
oracle/_build/libtgx_oracle.so).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the reference's native CPU
forward of the sum reducer, timed by bench.py as a CPU baseline and checked
against ref.sum_fwd by tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "_build" / "libtgx_oracle.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
        _lib = ctypes.CDLL(str(_LIB_PATH))
        p = ctypes.c_void_p
        _lib.tgx_oracle_csr_sum_fwd.argtypes = [p, p, p, p, p, ctypes.c_int64, ctypes.c_int64,
                                                ctypes.c_int]
        _lib.tgx_oracle_csr_sum_fwd.restype = ctypes.c_int
        _lib.tgx_oracle_csr_sum_bwd_lowered.argtypes = [p] * 8 + [ctypes.c_int64] * 3
        _lib.tgx_oracle_csr_sum_bwd_lowered.restype = ctypes.c_int
    return _lib


def csr_sum_fwd(row_ptr, col_idx, x, w, threads=1, out=None):
    """out[i, :] = sum_e w[e] * x[col[e], :] over row i's CSR edges, fp32,
    sequential per (row, feature) in stored edge order, the output elements
    split into `threads` contiguous chunks (compiler_module.cpp:2127-2139)."""
    row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int64)
    col_idx = np.ascontiguousarray(col_idx, dtype=np.int64)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(np.asarray(w).reshape(-1), dtype=np.float32)
    n_dst = row_ptr.size - 1
    F = int(np.prod(x.shape[1:])) if x.ndim > 1 else 1
    if out is None:
        out = np.empty((n_dst, *x.shape[1:]), dtype=np.float32)
    rc = lib().tgx_oracle_csr_sum_fwd(row_ptr.ctypes.data, col_idx.ctypes.data, x.ctypes.data,
                                      w.ctypes.data, out.ctypes.data, n_dst, F, int(threads))
    if rc != 0:
        raise RuntimeError(f"tgx_oracle_csr_sum_fwd failed ({rc})")
    return out


def csr_sum_bwd_lowered(row_ptr, col_idx, x, w, dout):
    """(dx, dw) of the weighted sum by the reference runtime's lowered native
    backward (LowerTensorToCPU.cpp:608-670): a select chain over every row per
    message element, then a scan over every edge per dx element.  Sequential;
    only for small graphs (O(E * N * F))."""
    row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int64)
    col_idx = np.ascontiguousarray(col_idx, dtype=np.int64)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(np.asarray(w).reshape(-1), dtype=np.float32)
    dout = np.ascontiguousarray(dout, dtype=np.float32)
    n_dst, n_src, F = row_ptr.size - 1, x.shape[0], x.shape[1]
    dx = np.empty((n_src, F), dtype=np.float32)
    dw = np.empty(col_idx.size, dtype=np.float32)
    scratch = np.empty((col_idx.size, F), dtype=np.float32)
    rc = lib().tgx_oracle_csr_sum_bwd_lowered(
        row_ptr.ctypes.data, col_idx.ctypes.data, x.ctypes.data, w.ctypes.data,
        dout.ctypes.data, dx.ctypes.data, dw.ctypes.data, scratch.ctypes.data, n_dst, n_src, F)
    if rc != 0:
        raise RuntimeError(f"tgx_oracle_csr_sum_bwd_lowered failed ({rc})")
    return dx, dw
