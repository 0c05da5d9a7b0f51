"""The ``quantibbler_kernels`` PyO3 face, on libqbk.

Same names, arguments, wire forms and error texts as the reference module
(crates/quantibbler-kernels/src/lib.rs:94-402), so
``src/quantibbler/kernels/__init__.py`` (which picks the extension by module
name and ``hasattr``) runs unchanged when this module is importable as
``quantibbler_kernels``:

    import sys, quantibbler_amd.kernels as k
    sys.modules["quantibbler_kernels"] = k

The packed products run on the GPU (a process-wide GpuContext on device 0);
pack_bits / unpack_bits / sign_estimate and joint_itq (the compressor's
alternating Procrustes) run in libqbk's host code, as the reference's do.
Errors raise ValueError subclasses (lib.rs:34-36 maps KernelError to
ValueError).
"""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np

from . import _lib
from ._lib import KernelError, check

__all__ = [
    "backend_version", "pack_bits", "unpack_bits", "sign_estimate", "packed_matvec",
    "packed_matmul", "packed_matvec_dtype", "packed_matmul_dtype", "joint_itq",
]

_ctx = None
_ctx_lock = threading.Lock()


def _context():
    global _ctx
    with _ctx_lock:
        if _ctx is None:
            from .gpu import GpuContext
            _ctx = GpuContext(0)
        return _ctx


def _rows_cols(shape):
    """lib.rs:67-72: flatten any dimensionality to rows x last axis."""
    n_cols = shape[-1] if len(shape) else 0
    n_rows = int(np.prod(shape[:-1], dtype=np.int64)) if len(shape) else 0
    return n_rows, n_cols


def backend_version() -> str:
    """lib.rs:94-97."""
    return _lib.load().qbk_backend_version().decode()


def _fmt_f64(v: float) -> str:
    return repr(float(v))


def pack_bits(factor) -> np.ndarray:
    """lib.rs:100-126: +-1 factor (float64 or int8, any dim) -> uint8 bitplanes."""
    a = np.asarray(factor)
    if a.dtype != np.int8:
        a = np.asarray(a, dtype=np.float64)
    n_rows, n_cols = _rows_cols(a.shape)
    flat = a.ravel()
    bad = np.flatnonzero((flat != 1) & (flat != -1))
    if bad.size:
        raise KernelError(
            "pack_bits expects values in {-1, +1}; got " + _fmt_f64(float(flat[bad[0]])))
    f8 = np.ascontiguousarray(flat, dtype=np.int8)
    n_words = (n_cols + 7) // 8
    out = np.zeros((n_rows, n_words), dtype=np.uint8)
    check(_lib.load().qbk_pack_bits(f8.ctypes.data, f8.size, n_rows, n_cols, out.ctypes.data))
    return out


def unpack_bits(packed, n_bits: int, dtype: str) -> np.ndarray:
    """lib.rs:129-156."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n_rows, n_words = _rows_cols(p.shape)
    if n_bits > n_words * 8:
        raise KernelError(
            f"n_bits={n_bits} exceeds the packed width {n_words} ({n_words * 8} bits)")
    out = np.zeros((n_rows, n_bits), dtype=np.int8)
    check(_lib.load().qbk_unpack_bits(p.ctypes.data, p.size, n_rows, n_bits, out.ctypes.data))
    if dtype == "int8":
        return out
    if dtype == "float64":
        return out.astype(np.float64)
    raise KernelError(f'unpack_bits dtype must be \'int8\' or \'float64\', got "{dtype}"')


def sign_estimate(x) -> np.ndarray:
    """lib.rs:159-171: int8 sign, exact zeros (and -0.0) -> +1."""
    a = np.ascontiguousarray(x, dtype=np.float64).ravel()
    out = np.zeros(a.size, dtype=np.int8)
    _lib.load().qbk_sign_estimate(a.ctypes.data, a.size, out.ctypes.data)
    return out


def _dtype_tag(dtype: str) -> int:
    v = C.c_int()
    check(_lib.load().qbk_dtype_from_name(str(dtype).encode(), C.byref(v)))
    return v.value


_NP = {_lib.QBK_F64: np.float64, _lib.QBK_F32: np.float32, _lib.QBK_BF16: np.uint16}
_NAME = {_lib.QBK_F64: "float64", _lib.QBK_F32: "float32", _lib.QBK_BF16: "bfloat16"}


def _matvec(packed, n_bits, vec, tag):
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n_rows, _ = _rows_cols(p.shape)
    v = np.ascontiguousarray(vec, dtype=_NP[tag]).ravel()
    return _context().packed_matvec(p, n_rows, int(n_bits), v, _NAME[tag])


def _matmul(packed, n_bits, mat, tag):
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n_rows, _ = _rows_cols(p.shape)
    m = np.ascontiguousarray(mat, dtype=_NP[tag])
    n_cols = m.shape[-1] if m.ndim else 0
    return _context().packed_matmul(p, n_rows, int(n_bits), m.ravel(), n_cols, _NAME[tag])


def packed_matvec(packed, n_bits: int, vec) -> np.ndarray:
    """lib.rs:174-186 (float64)."""
    return _matvec(packed, n_bits, vec, _lib.QBK_F64)


def packed_matmul(packed, n_bits: int, mat) -> np.ndarray:
    """lib.rs:189-208 (float64)."""
    return _matmul(packed, n_bits, mat, _lib.QBK_F64)


def packed_matvec_dtype(packed, n_bits: int, vec, dtype: str) -> np.ndarray:
    """lib.rs:293-321: the tag is resolved before the operand is touched."""
    return _matvec(packed, n_bits, vec, _dtype_tag(dtype))


def packed_matmul_dtype(packed, n_bits: int, mat, dtype: str) -> np.ndarray:
    """lib.rs:326-382."""
    return _matmul(packed, n_bits, mat, _dtype_tag(dtype))


def joint_itq(u_hat, v_hat, *, max_iter=None, tol=None, seed=None):
    """lib.rs:197-235: joint_itq over Z = [u_hat; v_hat] (core.rs:318-424)
    -> (u_t int8 (dout, r), v_t int8 (din, r), n_iter, converged)."""
    u = np.ascontiguousarray(u_hat, dtype=np.float64)
    v = np.ascontiguousarray(v_hat, dtype=np.float64)
    dout, rank = _rows_cols(u.shape)
    din, rank_v = _rows_cols(v.shape)
    if rank != rank_v:
        raise KernelError(f"joint_itq rank mismatch: u_hat r={rank}, v_hat r={rank_v}")
    ut = np.zeros((dout, rank), np.int8)
    vt = np.zeros((din, rank), np.int8)
    n_iter, conv = C.c_size_t(), C.c_int()
    check(_lib.load().qbk_joint_itq(u.ctypes.data, u.size, v.ctypes.data, v.size, dout, din, rank,
                                    50 if max_iter is None else int(max_iter),
                                    1e-12 if tol is None else float(tol), 0 if seed is None else int(seed),
                                    ut.ctypes.data, vt.ctypes.data, C.byref(n_iter), C.byref(conv)))
    return ut, vt, int(n_iter.value), bool(conv.value)
