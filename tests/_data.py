"""Seeded synthetic inputs and the parity bar shared by the tests.

Inputs are generated on the CPU with numpy's PCG64 so the oracle and the GPU
see identical bits.  The bar: fp32/complex64
``max|got - ref| <= 1e-4 * max|ref|``; fp64/complex128 ``<= 1e-10 * max|ref|``;
int64 exact.  ``|.|`` is the complex modulus.
"""
from __future__ import annotations

import zlib

import numpy as np

REAL = {np.float32: np.float32, np.float64: np.float64, np.complex64: np.float32, np.complex128: np.float64}


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def seed_of(*key) -> int:
    """Process-independent seed for a test case (unlike hash(), never salted)."""
    return zlib.crc32(repr(key).encode())


def normal(g, shape, dtype):
    dtype = np.dtype(dtype)
    if dtype.kind == "c":
        return (g.standard_normal(shape) + 1j * g.standard_normal(shape)).astype(dtype)
    return g.standard_normal(shape).astype(dtype)


def coef(g, shape, dtype, rmax=0.99):
    """Stable scalar coefficients: U(-rmax, rmax) real, r e^{i theta} complex."""
    dtype = np.dtype(dtype)
    if dtype.kind == "c":
        r = g.uniform(0.5, rmax, shape)
        th = g.uniform(0, np.pi, shape)
        return (r * np.exp(1j * th)).astype(dtype)
    return g.uniform(-rmax, rmax, shape).astype(dtype)


def biquad_A(g, shape, dtype, rlo=0.5, rhi=0.98):
    """2x2 transposed-companion matrices [[-a1, 1], [-a2, 0]] of stable biquads.

    Poles r e^{+-i theta}: a1 = -2 r cos(theta), a2 = r^2 (the TDF-II state
    matrix that philtorch's lfilter builds, philtorch/lti/filtering.py:304-317).
    For complex dtypes a random phase is applied to the whole matrix.
    """
    dtype = np.dtype(dtype)
    r = g.uniform(rlo, rhi, shape)
    th = g.uniform(0, np.pi, shape)
    a1, a2 = -2 * r * np.cos(th), r * r
    A = np.zeros(shape + (2, 2))
    A[..., 0, 0] = -a1
    A[..., 0, 1] = 1.0
    A[..., 1, 0] = -a2
    if dtype.kind == "c":
        ph = np.exp(1j * g.uniform(-0.3, 0.3, shape))[..., None, None]
        return (A * ph).astype(dtype)
    return A.astype(dtype)


def stable_matrix(g, shape, M, dtype, rmax=0.95):
    """Random M x M matrices (complex where dtype is) scaled to spectral norm
    U(0.5, rmax), so that every step contracts the state."""
    dtype = np.dtype(dtype)
    A = g.standard_normal(shape + (M, M))
    if dtype.kind == "c":
        A = A + 1j * g.standard_normal(shape + (M, M))
    norm = np.linalg.norm(A, ord=2, axis=(-2, -1))[..., None, None]
    return (A / norm * g.uniform(0.5, rmax, shape)[..., None, None]).astype(dtype)


def tol(dtype) -> float:
    dtype = np.dtype(dtype)
    if dtype in (np.dtype(np.float32), np.dtype(np.complex64)):
        return 1e-4
    if dtype in (np.dtype(np.float64), np.dtype(np.complex128)):
        return 1e-10
    return 0.0


def check(got, ref, name="", dtype=None, scale=None):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} != {ref.shape}"
    dtype = dtype or ref.dtype
    if np.dtype(dtype).kind in "iu":
        np.testing.assert_array_equal(got, ref, err_msg=name)
        return 0.0
    err = float(np.max(np.abs(got.astype(np.complex128) - ref.astype(np.complex128)))) if ref.size else 0.0
    own = float(np.max(np.abs(ref))) if ref.size else 0.0
    scale = own if scale is None else max(own, float(scale))
    bound = tol(dtype) * max(scale, np.finfo(np.float64).tiny)
    assert err <= bound, f"{name}: max|d|={err:.3e} > {tol(dtype):.0e} * max|ref| ({scale:.3e})"
    return err / max(scale, 1e-300)


def sos_coefs(g, lead, S, dtype, rlo=0.5, rhi=0.95, rz=1.2):
    """Second-order sections (b0, b1, b2, 1, a1, a2) of shape lead + (S, 6):
    poles r e^{+-i theta}, r ~ U(rlo, rhi), zeros r_z e^{+-i phi},
    r_z ~ U(0, rz), gain b0 ~ U(0.5, 1.5) (the C4 recipe of the benchmark)."""
    shape = tuple(lead) + (S,)
    r, th = g.uniform(rlo, rhi, shape), g.uniform(0, np.pi, shape)
    z, ph = g.uniform(0, rz, shape), g.uniform(0, np.pi, shape)
    k = g.uniform(0.5, 1.5, shape)
    sos = np.stack([k, -2 * z * np.cos(ph) * k, z * z * k, np.ones(shape), -2 * r * np.cos(th), r * r], axis=-1)
    return sos.astype(dtype)


def ba_coefs(g, lead, order, dtype, rlo=0.5, rhi=0.95):
    """A filter of the given order as philtorch's (b, a): b lead + (order + 1,),
    a lead + (order,) after the leading 1.  The product of order // 2
    sections of sos_coefs and, for an odd order, a first-order section with a
    real pole of radius U(rlo, rhi) and either sign, a real zero and gain."""
    lead = tuple(lead)
    n = int(np.prod(lead)) if lead else 1
    sos = sos_coefs(g, (n,), order // 2, np.float64, rlo, rhi).reshape(n, order // 2, 6)
    p = g.uniform(rlo, rhi, n) * np.where(g.uniform(size=n) < 0.5, -1.0, 1.0)
    z, k = g.uniform(-1.2, 1.2, n), g.uniform(0.5, 1.5, n)
    bs, as_ = [], []
    for r in range(n):
        bn, ad = np.ones(1), np.ones(1)
        for s in range(order // 2):
            bn, ad = np.convolve(bn, sos[r, s, :3]), np.convolve(ad, sos[r, s, 3:])
        if order % 2:
            bn, ad = np.convolve(bn, [k[r], -k[r] * z[r]]), np.convolve(ad, [1.0, -p[r]])
        bs.append(bn)
        as_.append(ad[1:])
    b = np.array(bs).reshape(lead + (order + 1,))
    a = np.array(as_).reshape(lead + (order,))
    return b.astype(dtype), a.astype(dtype)
