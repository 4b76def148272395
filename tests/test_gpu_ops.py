"""GPU parity of the philtorch ops (HIP kernels) against the CPU oracle.

Every case draws seeded inputs on the CPU, runs the op on cuda:0 and the
oracle (a restatement of philtorch's CPU extension and backward closures) on
the same bits, and applies the north-star bar from tests/_data.py.  Shapes
cover single steps, tile edges (tiles are 512..8192 steps), partial tiles,
T not divisible by the vector width, shared coefficients and rows long enough
for look-back windows of more than 64 predecessor tiles.
"""
import numpy as np
import pytest

from tests import _data as D

pytestmark = pytest.mark.gpu

FLOATS = [np.float32, np.float64, np.complex64, np.complex128]
SHAPES = [(1, 1), (3, 1), (2, 5), (4, 4095), (4, 4096), (3, 4097), (2, 8192), (1, 8193), (2, 3 * 4096 + 17),
          (5, 20001)]


def _t(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _n(t):
    return t.detach().cpu().numpy()


# ----------------------------------------------------------------- recur (LPV scalar)
@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("shared", [False, True])
def test_recur_fwd_bwd(hip, dtype, shape, shared):
    import torch
    import oracle

    B, T = shape
    g = D.rng(D.seed_of(B, T, shared, np.dtype(dtype).str))
    A = D.coef(g, (T,) if shared else (B, T), dtype)
    zi = D.normal(g, (B,), dtype)
    x = D.normal(g, (B, T), dtype)
    gy = D.normal(g, (B, T), dtype)
    y_ref = oracle.recur(A, zi, x)
    y = torch.ops.philtorch.recur(_t(A), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    gA_ref, gzi_ref, gx_ref = oracle.recur_bwd(A, zi, y_ref, gy)
    gA, gzi, gx = torch.ops.philtorch.recur_backward(_t(A), _t(zi), y, _t(gy))
    D.check(_n(gx), gx_ref, "grad_x")
    D.check(_n(gzi), gzi_ref, "grad_zi")
    D.check(_n(gA), gA_ref, "grad_A")


def test_recur_many_tiles(hip):
    """One row of 2**20 steps: 256 tiles, look-back across several windows."""
    import torch
    import oracle

    g = D.rng(11)
    B, T = 2, 1 << 20
    A = (0.999 * np.tanh(2 * g.standard_normal((B, T)))).astype(np.float32)
    zi = D.normal(g, (B,), np.float32)
    x = D.normal(g, (B, T), np.float32)
    gy = D.normal(g, (B, T), np.float32)
    y_ref = oracle.recur(A, zi, x)
    y = torch.ops.philtorch.recur(_t(A), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    ref = oracle.recur_bwd(A, zi, y_ref, gy)
    got = torch.ops.philtorch.recur_backward(_t(A), _t(zi), y, _t(gy))
    for name, a, b in zip(("grad_A", "grad_zi", "grad_x"), got, ref):
        D.check(_n(a), b, name)


# ----------------------------------------------------------------- lti_recur
@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("shared", [False, True])
def test_lti_recur_fwd_bwd(hip, dtype, shape, shared):
    import torch
    import oracle

    B, T = shape
    g = D.rng(D.seed_of('lti', B, T, shared, np.dtype(dtype).str))
    a = D.coef(g, (1,) if shared else (B,), dtype)
    if shared and B == 1:
        a = a.reshape(())  # 0-D scalar form
    zi = D.normal(g, (B,), dtype)
    x = D.normal(g, (B, T), dtype)
    gy = D.normal(g, (B, T), dtype)
    y_ref = oracle.lti_recur(a, zi, x)
    y = torch.ops.philtorch.lti_recur(_t(a), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    ga_ref, gzi_ref, gx_ref = oracle.lti_recur_bwd(a, zi, y_ref, gy)
    ga, gzi, gx = torch.ops.philtorch.lti_recur_backward(_t(a), _t(zi), y, _t(gy))
    D.check(_n(gx), gx_ref, "grad_x")
    D.check(_n(gzi), gzi_ref, "grad_zi")
    D.check(_n(ga).reshape(-1), ga_ref.reshape(-1), "grad_a")


# ----------------------------------------------------------------- recur2 / lti_recur2
SHAPES2 = [(1, 1), (2, 7), (3, 2047), (3, 2048), (2, 2049), (2, 5003)]


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", SHAPES2)
@pytest.mark.parametrize("shared", [False, True])
def test_recur2_fwd_bwd(hip, dtype, shape, shared):
    import torch
    import oracle

    B, T = shape
    g = D.rng(D.seed_of('recur2', B, T, shared, np.dtype(dtype).str))
    A = D.biquad_A(g, (T,) if shared else (B, T), dtype)
    zi = D.normal(g, (B, 2), dtype)
    x = D.normal(g, (B, T, 2), dtype)
    gy = D.normal(g, (B, T, 2), dtype)
    y_ref = oracle.recurN(A, zi, x)
    y = torch.ops.philtorch.recur2(_t(A), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    ref = oracle.recurN_bwd(A, zi, y_ref, gy)
    got = torch.ops.philtorch.recurN_backward(_t(A), _t(zi), y, _t(gy))
    for name, a, b in zip(("grad_A", "grad_zi", "grad_x"), got, ref):
        D.check(_n(a), b, name)


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", SHAPES2)
@pytest.mark.parametrize("shared", [False, True])
def test_lti_recur2_fwd_bwd(hip, dtype, shape, shared):
    import torch
    import oracle

    B, T = shape
    g = D.rng(D.seed_of('lti2', B, T, shared, np.dtype(dtype).str))
    A = D.biquad_A(g, () if shared else (B,), dtype)
    zi = D.normal(g, (B, 2), dtype)
    x = D.normal(g, (B, T, 2), dtype)
    gy = D.normal(g, (B, T, 2), dtype)
    y_ref = oracle.lti_recurN(A, zi, x)
    y = torch.ops.philtorch.lti_recur2(_t(A), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    ref = oracle.lti_recurN_bwd(A, zi, y_ref, gy)
    got = torch.ops.philtorch.lti_recurN_backward(_t(A), _t(zi), y, _t(gy))
    for name, a, b in zip(("grad_A", "grad_zi", "grad_x"), got, ref):
        D.check(_n(a), b, name)


# ----------------------------------------------------------------- recurN / lti_recurN, M = 3, 4
SHAPES_N = [(1, 1), (2, 7), (3, 1025), (2, 3001)]


@pytest.mark.parametrize("M", [3, 4])
@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", SHAPES_N)
@pytest.mark.parametrize("shared", [False, True])
def test_recurN_order_fwd_bwd(hip, M, dtype, shape, shared):
    import torch
    import oracle

    B, T = shape
    g = D.rng(D.seed_of('recurN', M, B, T, shared, np.dtype(dtype).str))
    A = D.stable_matrix(g, (T,) if shared else (B, T), M, dtype)
    zi = D.normal(g, (B, M), dtype)
    x = D.normal(g, (B, T, M), dtype)
    gy = D.normal(g, (B, T, M), dtype)
    y_ref = oracle.recurN(A, zi, x)
    y = torch.ops.philtorch.recurN(_t(A), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    ref = oracle.recurN_bwd(A, zi, y_ref, gy)
    got = torch.ops.philtorch.recurN_backward(_t(A), _t(zi), y, _t(gy))
    for name, a, b in zip(("grad_A", "grad_zi", "grad_x"), got, ref):
        D.check(_n(a), b, name)


@pytest.mark.parametrize("M", [3, 4])
@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", SHAPES_N)
@pytest.mark.parametrize("shared", [False, True])
def test_lti_recurN_order_fwd_bwd(hip, M, dtype, shape, shared):
    import torch
    import oracle

    B, T = shape
    g = D.rng(D.seed_of('lti_recurN', M, B, T, shared, np.dtype(dtype).str))
    A = D.stable_matrix(g, () if shared else (B,), M, dtype)
    zi = D.normal(g, (B, M), dtype)
    x = D.normal(g, (B, T, M), dtype)
    gy = D.normal(g, (B, T, M), dtype)
    y_ref = oracle.lti_recurN(A, zi, x)
    y = torch.ops.philtorch.lti_recurN(_t(A), _t(zi), _t(x))
    D.check(_n(y), y_ref, "y")
    ref = oracle.lti_recurN_bwd(A, zi, y_ref, gy)
    got = torch.ops.philtorch.lti_recurN_backward(_t(A), _t(zi), y, _t(gy))
    for name, a, b in zip(("grad_A", "grad_zi", "grad_x"), got, ref):
        D.check(_n(a), b, name)


def test_recurN_order_above_native_raises(hip):
    import torch

    A = torch.zeros(2, 5, 5, 5, device="cuda")
    with pytest.raises(RuntimeError, match="up to M = 4"):
        torch.ops.philtorch.recurN(A, torch.zeros(2, 5, device="cuda"), torch.zeros(2, 5, 5, device="cuda"))


def test_fibonacci_int64(hip):
    """README known answer (philtorch README.md:143-159) through lti_recur2 in int64."""
    import torch

    A = torch.tensor([[1, 1], [1, 0]], dtype=torch.long, device="cuda")
    zi = torch.zeros(1, 2, dtype=torch.long, device="cuda")
    x = torch.zeros(1, 10, 2, dtype=torch.long, device="cuda")
    x[0, 0, 0] = 1
    y = torch.ops.philtorch.lti_recur2(A, zi, x)
    assert y[0, :, 0].tolist() == [1, 1, 2, 3, 5, 8, 13, 21, 34, 55]


def test_recurN_scalar_route(hip):
    """recurN with 1x1 matrices equals the dedicated scalar op."""
    import torch
    import oracle

    g = D.rng(5)
    B, T = 3, 9000
    A = D.coef(g, (B, T), np.float64)
    zi = D.normal(g, (B,), np.float64)
    x = D.normal(g, (B, T), np.float64)
    y = torch.ops.philtorch.recurN(_t(A)[..., None, None], _t(zi)[:, None], _t(x)[..., None])
    D.check(_n(y)[..., 0], oracle.recur(A, zi, x), "y")
