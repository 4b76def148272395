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


# ------------------------------------------------------------------ SOS cascade
# philtorch has no cascade op: a cascade of second-order sections is one
# lfilter(form="tdf2") per section.  Each section is the state-space model
# _ssm_lfilter builds (philtorch/lti/filtering.py:273-333; companion matrix
# philtorch/mat.py:42-62) run through state_space with out_idx=0
# (philtorch/lti/ssm.py:386-510): Bx = x Bv, h = lti_recurN(A, zi, Bx),
# y = [zi.0, h[:-1].0] + b0 x, zf = h[-1].  The backward is the chain rule of
# that graph around _lti_recurN_backward (philtorch/__init__.py:76-112).
def _tdf2_section(sos_s):
    """(A [R,2,2], Bv [R,2], b0 [R], a [R,2]) of sections sos_s [R,6] with a0 = 1:
    A = companion(a).mT = [[-a1, 1], [-a2, 0]], Bv = b[1:] - b0 a."""
    b0, b1, b2, a1, a2 = sos_s[:, 0], sos_s[:, 1], sos_s[:, 2], sos_s[:, 4], sos_s[:, 5]
    A = np.zeros((sos_s.shape[0], 2, 2), dtype=sos_s.dtype)
    A[:, 0, 0] = -a1
    A[:, 0, 1] = 1
    A[:, 1, 0] = -a2
    Bv = np.stack([b1 - b0 * a1, b2 - b0 * a2], axis=-1)
    return A, Bv, b0, np.stack([a1, a2], axis=-1)


def _sos_rows(sos, B):
    """sos [S,6] (shared) or [B,S,6] -> per-row view [B,S,6] and the shared flag."""
    sos = np.asarray(sos)
    if sos.ndim == 2:
        return np.broadcast_to(sos, (B,) + sos.shape), True
    return sos, False


def _sos_section_fwd(A, Bv, b0, zi, u, nthreads):
    Bx = u[..., None] * Bv[:, None, :]
    h = lti_recurN(A, zi, Bx, nthreads)
    y = np.concatenate([zi[:, None, 0], h[:, :-1, 0]], axis=1) + b0[:, None] * u
    return y, h


def sosfilt(sos, x, zi=None, nthreads=None):
    """Cascade of second-order sections, sos [S,6] or [B,S,6] with a0 = 1;
    x [B,T]; zi [B,S,2] or None.  Returns (y [B,T], zf [B,S,2])."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    B, T = x.shape
    rows, _ = _sos_rows(_c(sos, dt), B)
    S = rows.shape[1]
    zi = np.zeros((B, S, 2), dtype=dt) if zi is None else _c(zi, dt)
    zf = np.empty((B, S, 2), dtype=dt)
    u = x
    for s in range(S):
        A, Bv, b0, _ = _tdf2_section(_c(rows[:, s], dt))
        u, h = _sos_section_fwd(A, Bv, b0, _c(zi[:, s], dt), u, nthreads)
        zf[:, s] = h[:, -1] if T > 0 else zi[:, s]
    return u, zf


def sosfilt_bwd(sos, x, zi, gy, gzf=None, nthreads=None):
    """Backward of sosfilt for upstream gradients gy [B,T] and gzf [B,S,2]
    (None = 0).  Returns (grad_sos, grad_zi, grad_x); grad_sos has sos's
    shape (summed over rows when shared; the a0 column is 0)."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    B, T = x.shape
    rows, shared = _sos_rows(_c(sos, dt), B)
    S = rows.shape[1]
    zi = np.zeros((B, S, 2), dtype=dt) if zi is None else _c(zi, dt)
    gzf = np.zeros((B, S, 2), dtype=dt) if gzf is None else _c(gzf, dt)
    secs, ins, hs = [], [], []
    u = x
    for s in range(S):
        sec = _tdf2_section(_c(rows[:, s], dt))
        ins.append(u)
        u, h = _sos_section_fwd(*sec[:3], _c(zi[:, s], dt), u, nthreads)
        secs.append(sec)
        hs.append(h)
    g = _c(gy, dt)
    gsos = np.zeros((B, S, 6), dtype=dt)
    gzi = np.zeros((B, S, 2), dtype=dt)
    for s in reversed(range(S)):
        A, Bv, b0, a = secs[s]
        u, h = ins[s], hs[s]
        # y = shift(h).0 + b0 u
        gh = np.zeros_like(h)
        gh[:, :-1, 0] = g[:, 1:]
        gh[:, -1] += gzf[:, s]
        gzi_s = np.zeros((B, 2), dtype=dt)
        gzi_s[:, 0] = g[:, 0]
        gb0 = np.sum(g * u, axis=1)
        gu = b0[:, None] * g
        gA, gz, gBx = lti_recurN_bwd(A, _c(zi[:, s], dt), h, gh, nthreads)
        gzi_s += gz
        gu = gu + np.sum(gBx * Bv[:, None, :], axis=-1)
        gBv = np.sum(gBx * u[..., None], axis=1)
        # Bv = b[1:] - b0 a;  A = [[-a1, 1], [-a2, 0]]
        gsos[:, s, 0] = gb0 - np.sum(a * gBv, axis=-1)
        gsos[:, s, 1] = gBv[:, 0]
        gsos[:, s, 2] = gBv[:, 1]
        gsos[:, s, 4] = -gA[:, 0, 0] - b0 * gBv[:, 0]
        gsos[:, s, 5] = -gA[:, 1, 0] - b0 * gBv[:, 1]
        gzi[:, s] = gzi_s
        g = gu
    if shared:
        gsos = gsos.sum(axis=0)
    return gsos, gzi, g


# torch.nn.functional.pad mode -> numpy.pad mode
_NP_PAD = {"constant": "constant", "replicate": "edge", "reflect": "reflect", "circular": "wrap"}


def lfilter_zi(sos_rows):
    """Steady state of TDF-II biquads sos_rows [R,6] (a0 = 1) for a unit
    input: solve((I - A), Bv) as philtorch's lfilter_zi does
    (philtorch/lti/filtering.py:107-142, transpose=True)."""
    A, Bv, _, _ = _tdf2_section(np.asarray(sos_rows))
    I_minus_A = np.eye(2, dtype=A.dtype)[None] - A
    return np.linalg.solve(I_minus_A, Bv[..., None])[..., 0]


def filtfilt(sos, x, padmode="replicate", padlen=None, nthreads=None):
    """philtorch.lti.filtfilt of one biquad per row
    (philtorch/lti/filtering.py:413-484): sos [6] (shared) or [B,6] with
    a0 = 1; x [B,T].  Pads by `padlen` (default 3 * ntaps = 9) with
    torch.nn.functional.pad's `padmode` (None: no padding), filters forward
    from lfilter_zi * ext[:, 0], filters the reversed output from
    lfilter_zi * y[:, -1], trims and flips back; each pass is one
    lfilter(tdf2) (sosfilt with one section)."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    B, T = x.shape
    rows = np.broadcast_to(_c(sos, dt), (B, 6)) if np.ndim(sos) == 1 else _c(sos, dt)
    edge = 0 if padmode is None else (9 if padlen is None else int(padlen))
    assert T > edge, f"Input signal length {T} must be greater than pad length {edge}."
    ext = np.pad(x, ((0, 0), (edge, edge)), mode=_NP_PAD[padmode]) if edge > 0 else x
    ext = np.ascontiguousarray(ext)
    zi = lfilter_zi(rows).astype(dt)
    sec = np.ascontiguousarray(rows[:, None, :])
    y, _ = sosfilt(sec, ext, np.ascontiguousarray((zi * ext[:, :1])[:, None, :]), nthreads)
    yr = np.ascontiguousarray(y[:, ::-1])
    y, _ = sosfilt(sec, yr, np.ascontiguousarray((zi * yr[:, :1])[:, None, :]), nthreads)
    if edge > 0:
        y = y[:, edge:-edge]
    return np.ascontiguousarray(y[:, ::-1])



def lpv_state_space(A, x, B=None, C=None, D=None, zi=None, out_idx=None, nthreads=None):
    """philtorch.lpv.state_space for a 2D input and a single output
    (philtorch/lpv/ssm.py:337-581) on operands broadcast to per row and
    step: A [T,M,M] or [B,T,M,M]; B, C [1|B, 1|T, M] (B None: the input
    enters state 0; C None: state out_idx); D [1|B, 1|T] or None.  B x, the
    LPV scan recurN, the state sequence shifted by one step behind zi, then
    y = c[t] . h + d[t] x.  Returns (y [B,T], zf [B,M])."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    Bn, T = x.shape
    M = np.shape(A)[-1]
    A = _c(np.broadcast_to(A, (Bn, T, M, M)), dt)
    zi = np.zeros((Bn, M), dtype=dt) if zi is None else _c(np.broadcast_to(zi, (Bn, M)), dt)
    if B is None:
        Bx = np.zeros((Bn, T, M), dtype=dt)
        Bx[..., 0] = x
    else:
        Bx = x[..., None] * np.broadcast_to(np.asarray(B, dtype=dt), (Bn, T, M))
    h = recurN(A, zi, _c(Bx, dt), nthreads)
    zf = h[:, -1] if T > 0 else zi.copy()
    hprev = np.concatenate([zi[:, None, :], h[:, :-1]], axis=1)[:, :T]
    if C is None:
        y = hprev[..., out_idx].copy()
    else:
        y = np.einsum("btm,btm->bt", hprev, np.broadcast_to(np.asarray(C, dtype=dt), (Bn, T, M)))
    if D is not None:
        y = y + np.broadcast_to(np.asarray(D, dtype=dt), (Bn, T)) * x
    return _c(y, dt), _c(zf, dt)


def lpv_state_space_mimo(A, x, B, C, D=None, zi=None, nthreads=None):
    """philtorch.lpv.state_space with matrix operands constant in time
    (philtorch/lpv/ssm.py:337-581 for a 3D input): x [Bn,T,F]; A [T,M,M] or
    [Bn,T,M,M]; B [M,F] or [Bn,M,F]; C [P,M] or [Bn,P,M]; D None, [P,F] or
    [Bn,P,F].  Bx[t] = B x[t] (:413-454), the LPV scan recurN, the state
    sequence shifted one step behind zi (:462-474), then y = C h + D x
    (:480-577).  Returns (y [Bn,T,P], zf [Bn,M])."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    Bn, T, F = x.shape
    M = np.shape(A)[-1]
    A = _c(np.broadcast_to(A, (Bn, T, M, M)), dt)
    Bm = np.broadcast_to(np.asarray(B, dtype=dt), (Bn, M, F))
    Cm = np.asarray(C, dtype=dt)
    P = Cm.shape[-2]
    Cm = np.broadcast_to(Cm, (Bn, P, M))
    zi = np.zeros((Bn, M), dtype=dt) if zi is None else _c(np.broadcast_to(zi, (Bn, M)), dt)
    Bx = np.einsum("bmf,btf->btm", Bm, x)
    h = recurN(A, zi, _c(Bx, dt), nthreads)
    zf = h[:, -1] if T > 0 else zi.copy()
    hprev = np.concatenate([zi[:, None, :], h[:, :-1]], axis=1)[:, :T]
    y = np.einsum("bpm,btm->btp", Cm, hprev)
    if D is not None:
        y = y + np.einsum("bpf,btf->btp", np.broadcast_to(np.asarray(D, dtype=dt), (Bn, P, F)), x)
    return _c(y, dt), _c(zf, dt)


def _tdf2_companion(b, a):
    """TDF-II model of lfilter(b, a) per row (philtorch/lti/filtering.py:
    107-142 and :273-333, transpose=True): b [R,nb], a [R,na] (after the
    leading 1) zero-padded to order M = max(nb - 1, na); A = companion(a)^T
    [R,M,M], g = b[1:] - b[0] a [R,M], b0 [R]; y = h[0] + b0 u."""
    b = np.asarray(b, np.float64)
    a = np.asarray(a, np.float64)
    M = max(b.shape[-1] - 1, a.shape[-1])
    bp = np.zeros(b.shape[:-1] + (M + 1,))
    bp[..., : b.shape[-1]] = b
    ap = np.zeros(a.shape[:-1] + (M,))
    ap[..., : a.shape[-1]] = a
    A = np.zeros(a.shape[:-1] + (M, M))
    A[..., :, 0] = -ap
    A[..., np.arange(M - 1), np.arange(1, M)] = 1.0
    return A, bp[..., 1:] - bp[..., :1] * ap, bp[..., 0]


def lfilter_zi_ba(b, a):
    """lfilter_zi(a, b) of philtorch (filtering.py:107-142, transpose=True):
    solve(I - A, g) on the TDF-II model of each row of b [R,nb], a [R,na]."""
    A, g, _ = _tdf2_companion(b, a)
    return np.linalg.solve(np.eye(A.shape[-1]) - A, g[..., None])[..., 0]


def filtfilt_ba(b, a, x, padmode="replicate", padlen=None, nthreads=None):
    """philtorch.lti.filtfilt (philtorch/lti/filtering.py:413-484) for a
    filter of any order: b [nb] or [B,nb], a [na] or [B,na] (after the
    leading 1), x [B,T].  Pads by `padlen` (default 3 * max(nb, na + 1)) with
    F.pad's `padmode` (None: no padding), runs lfilter(tdf2) -- the TDF-II
    model through lti_state_space -- from lfilter_zi * ext[:, 0], again over
    the reversed output from lfilter_zi * y[:, -1], trims and flips back."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    B, T = x.shape
    b = np.broadcast_to(np.asarray(b, np.float64), (B, np.shape(b)[-1])).astype(dt).astype(np.float64)
    a = np.broadcast_to(np.asarray(a, np.float64), (B, np.shape(a)[-1])).astype(dt).astype(np.float64)
    ntaps = max(b.shape[-1], a.shape[-1] + 1)
    edge = 0 if padmode is None else (3 * ntaps if padlen is None else int(padlen))
    assert T > edge, f"Input signal length {T} must be greater than pad length {edge}."
    ext = np.pad(x, ((0, 0), (edge, edge)), mode=_NP_PAD[padmode]) if edge > 0 else x
    ext = np.ascontiguousarray(ext)
    A, g, b0 = _tdf2_companion(b, a)
    M = A.shape[-1]
    zi = lfilter_zi_ba(b, a)
    e0 = np.eye(M)[0]
    A, g, b0, zi = (v.astype(dt) for v in (A, g, b0, zi))
    y, _ = lti_state_space(A, ext, B=g, C=e0, D=b0, zi=zi * ext[:, :1], nthreads=nthreads)
    yr = np.ascontiguousarray(y[:, ::-1])
    y, _ = lti_state_space(A, yr, B=g, C=e0, D=b0, zi=zi * yr[:, :1], nthreads=nthreads)
    if edge > 0:
        y = y[:, edge:-edge]
    return np.ascontiguousarray(y[:, ::-1])


def lti_state_space_mimo(A, x, B, C, D=None, zi=None, nthreads=None):
    """philtorch.lti.state_space with matrix operands (philtorch/lti/ssm.py:
    386-589 for a 3D input (batch, time, features)): x [Bn,T,F]; A [M,M] or
    [Bn,M,M]; B [M,F] or [Bn,M,F]; C [P,M] or [Bn,P,M]; D None, [P,F] or
    [Bn,P,F].  Bx[t] = B x[t] (:478-482), the scan lti_recurN, the state
    sequence shifted one step behind zi (:493-504), then y = C h + D x
    (_ssm_C_D :513-589, its (_, M) / (batch, _, M) and (_, features) /
    (batch, _, features) branches).  Returns (y [Bn,T,P], zf [Bn,M])."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    Bn, T, F = x.shape
    A = _c(np.broadcast_to(A, (Bn,) + np.shape(A)[-2:]), dt)
    M = A.shape[-1]
    Bm = np.broadcast_to(np.asarray(B, dtype=dt), (Bn, M, F))
    Cm = np.asarray(C, dtype=dt)
    P = Cm.shape[-2]
    Cm = np.broadcast_to(Cm, (Bn, P, M))
    zi = np.zeros((Bn, M), dtype=dt) if zi is None else _c(np.broadcast_to(zi, (Bn, M)), dt)
    Bx = np.einsum("bmf,btf->btm", Bm, x)
    h = lti_recurN(A, zi, _c(Bx, dt), nthreads)
    zf = h[:, -1] if T > 0 else zi.copy()
    hprev = np.concatenate([zi[:, None, :], h[:, :-1]], axis=1)[:, :T]
    y = np.einsum("bpm,btm->btp", Cm, hprev)
    if D is not None:
        y = y + np.einsum("bpf,btf->btp", np.broadcast_to(np.asarray(D, dtype=dt), (Bn, P, F)), x)
    return _c(y, dt), _c(zf, dt)


def lti_state_space(A, x, B=None, C=None, D=None, zi=None, out_idx=None, nthreads=None):
    """philtorch.lti.state_space for a 2D input and a single output
    (philtorch/lti/ssm.py:386-589): Bx = x b (b an M-vector per row or shared;
    None = the input enters state 0, as _ext_ss_recur pads it), the scan
    lti_recurN, the state sequence shifted by one step behind zi, then
    y = C h + D x (C an M-vector per row or shared, or state out_idx; D one
    value or one per row).  Returns (y [B,T], zf [B,M])."""
    dt = np.asarray(x).dtype
    x = _c(x, dt)
    Bn, T = x.shape
    A = _c(np.broadcast_to(A, (Bn,) + np.shape(A)[-2:]), dt)
    M = A.shape[-1]
    zi = np.zeros((Bn, M), dtype=dt) if zi is None else _c(np.broadcast_to(zi, (Bn, M)), dt)
    if B is None:
        Bx = np.zeros((Bn, T, M), dtype=dt)
        Bx[..., 0] = x
    else:
        Bx = x[..., None] * np.broadcast_to(np.asarray(B, dtype=dt), (Bn, M))[:, None, :]
    h = lti_recurN(A, zi, _c(Bx, dt), nthreads)
    zf = h[:, -1] if T > 0 else zi.copy()
    hprev = np.concatenate([zi[:, None, :], h[:, :-1]], axis=1)[:, :T]
    if C is None:
        y = hprev[..., out_idx].copy()
    else:
        y = np.einsum("btm,bm->bt", hprev, np.broadcast_to(np.asarray(C, dtype=dt), (Bn, M)))
    if D is not None:
        y = y + np.broadcast_to(np.asarray(D, dtype=dt).reshape(-1), (Bn,))[:, None] * x
    return _c(y, dt), _c(zf, dt)
