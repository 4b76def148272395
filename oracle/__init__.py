"""CPU oracle — TEST INFRASTRUCTURE ONLY (ctypes over oracle/liboracle.so).

Restates philtorch's CPU extension and its backward closures (see the header
of phs_oracle.c for the file:line each function follows).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, always as the
checker or the timed CPU baseline, never as the thing measured on the GPU.

All functions take and return numpy arrays (C-contiguous) of one dtype among
float32, float64, complex64, complex128, int64.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_SUFFIX = {
    np.dtype(np.float32): "f32",
    np.dtype(np.float64): "f64",
    np.dtype(np.complex64): "c64",
    np.dtype(np.complex128): "c128",
    np.dtype(np.int64): "i64",
}

_lib = None


def build() -> str:
    """Compile liboracle.so with gcc (OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _threads(n):
    return ctypes.c_int(0 if n is None else n)


# ------------------------------------------------------------------ forward
def recurN(A, zi, x, nthreads=None):
    """philtorch::recurN / recur2 CPU (host_recurN.cpp:236-281).
    A [B,T,M,M] or shared [T,M,M]; zi [B,M]; x [B,T,M] -> y [B,T,M]."""
    dt = x.dtype
    x = _c(x, dt); zi = _c(zi, dt); A = _c(A, dt)
    B, T, M = x.shape
    y = np.empty_like(x)
    fn = getattr(lib(), f"oracle_recurN_{_SUFFIX[np.dtype(dt)]}")
    rc = fn(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(M), _ptr(A), ctypes.c_int(int(A.ndim == 4)),
            _ptr(zi), _ptr(x), _ptr(y), _threads(nthreads))
    assert rc == 0
    return y


def recur(A, zi, x, nthreads=None):
    """LPV scalar scan = recurN with 1x1 matrices. A [B,T] or [T]; zi [B]; x [B,T]."""
    A = np.asarray(A)
    y = recurN(A[..., None, None], np.asarray(zi)[:, None], np.asarray(x)[..., None], nthreads)
    return y[..., 0]


def lti_recurN(A, zi, x, nthreads=None):
    """philtorch::lti_recurN / lti_recur2 CPU (host_lti_recurN.cpp:5-108).
    A [B,M,M] or shared [M,M]; zi [B,M]; x [B,T,M]."""
    dt = x.dtype
    x = _c(x, dt); zi = _c(zi, dt); A = _c(A, dt)
    B, T, M = x.shape
    y = np.empty_like(x)
    fn = getattr(lib(), f"oracle_lti_recurN_{_SUFFIX[np.dtype(dt)]}")
    rc = fn(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(M), _ptr(A), ctypes.c_int(int(A.ndim == 3)),
            _ptr(zi), _ptr(x), _ptr(y), _threads(nthreads))
    assert rc == 0
    return y


def lti_recur(a, zi, x, nthreads=None):
    """philtorch::lti_recur CPU (host_lti_recur.cpp:42-80). a: [B] or one value."""
    dt = x.dtype
    x = _c(x, dt); zi = _c(zi, dt); a = _c(np.atleast_1d(a), dt)
    B, T = x.shape
    y = np.empty_like(x)
    fn = getattr(lib(), f"oracle_lti_recur_{_SUFFIX[np.dtype(dt)]}")
    rc = fn(ctypes.c_int64(B), ctypes.c_int64(T), _ptr(a), ctypes.c_int64(a.size), _ptr(zi), _ptr(x), _ptr(y),
            _threads(nthreads))
    assert rc == 0
    return y


# ------------------------------------------------------------------ backward
def recurN_bwd(A, zi, y, gy, nthreads=None):
    """_recurN_backward (philtorch/__init__.py:34-73) -> (grad_A, grad_zi, grad_x)."""
    dt = y.dtype
    A = _c(A, dt); zi = _c(zi, dt); y = _c(y, dt); gy = _c(gy, dt)
    B, T, M = y.shape
    gA = np.empty_like(A); gzi = np.empty_like(zi); gx = np.empty_like(y)
    fn = getattr(lib(), f"oracle_recurN_bwd_{_SUFFIX[np.dtype(dt)]}")
    rc = fn(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(M), _ptr(A), ctypes.c_int(int(A.ndim == 4)),
            _ptr(zi), _ptr(y), _ptr(gy), _ptr(gA), _ptr(gzi), _ptr(gx), _threads(nthreads))
    assert rc == 0
    return gA, gzi, gx


def recur_bwd(A, zi, y, gy, nthreads=None):
    """Scalar LPV backward: recurN_bwd with 1x1 matrices."""
    A = np.asarray(A)
    gA, gzi, gx = recurN_bwd(A[..., None, None], np.asarray(zi)[:, None], np.asarray(y)[..., None],
                             np.asarray(gy)[..., None], nthreads)
    return gA[..., 0, 0], gzi[:, 0], gx[..., 0]


def lti_recurN_bwd(A, zi, y, gy, nthreads=None):
    """_lti_recurN_backward (philtorch/__init__.py:76-112)."""
    dt = y.dtype
    A = _c(A, dt); zi = _c(zi, dt); y = _c(y, dt); gy = _c(gy, dt)
    B, T, M = y.shape
    gA = np.empty_like(A); gzi = np.empty_like(zi); gx = np.empty_like(y)
    fn = getattr(lib(), f"oracle_lti_recurN_bwd_{_SUFFIX[np.dtype(dt)]}")
    rc = fn(ctypes.c_int64(B), ctypes.c_int64(T), ctypes.c_int64(M), _ptr(A), ctypes.c_int(int(A.ndim == 3)),
            _ptr(zi), _ptr(y), _ptr(gy), _ptr(gA), _ptr(gzi), _ptr(gx), _threads(nthreads))
    assert rc == 0
    return gA, gzi, gx


def lti_recur_bwd(a, zi, y, gy, nthreads=None):
    """_lti_recur_backward (philtorch/__init__.py:115-148). grad_a has a's size."""
    dt = y.dtype
    a = _c(np.atleast_1d(a), dt); zi = _c(zi, dt); y = _c(y, dt); gy = _c(gy, dt)
    B, T = y.shape
    ga = np.empty_like(a); gzi = np.empty_like(zi); gx = np.empty_like(y)
    fn = getattr(lib(), f"oracle_lti_recur_bwd_{_SUFFIX[np.dtype(dt)]}")
    rc = fn(ctypes.c_int64(B), ctypes.c_int64(T), _ptr(a), ctypes.c_int64(a.size), _ptr(zi), _ptr(y), _ptr(gy),
            _ptr(ga), _ptr(gzi), _ptr(gx), _threads(nthreads))
    assert rc == 0
    return ga, gzi, gx
