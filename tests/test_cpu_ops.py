"""The CPU dispatch key of the philtorch ops (CPU only; no GPU needed).

torch.ops.philtorch.{recur2, recurN, lti_recur2, lti_recurN, lti_recur} on CPU
tensors run philtorch_amd's own CPU kernels (philtorch_amd/csrc/phs_cpu.hpp),
as the reference's CPU extension serves them (philtorch/csrc/host_recurN.cpp:
283-287, host_lti_recur.cpp:82-85, host_lti_recurN.cpp:110-114), so the
reference's backend indicators (philtorch/lpv/ssm.py:20-26, lti/ssm.py:13-25)
dispatch unchanged.  Pins:

* the golden vectors written by the reference's own CPU operators, bit for
  bit (the kernels keep the reference's loop order);
* the oracle (a separate restatement) at orders 1..5, every float dtype,
  shared and batched coefficients; the backward ops against the oracle's
  backward closures;
* the README Fibonacci known answer in int64;
* torch.library.opcheck on CPU tensors, and autograd (gradcheck) through the
  API Functions.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from tests import _data as D

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")
FLOATS = [np.float32, np.float64, np.complex64, np.complex128]


@pytest.fixture(scope="module")
def ops():
    import philtorch_amd

    philtorch_amd.require_extension()
    return torch.ops.philtorch


def _t(v):
    return torch.from_numpy(np.ascontiguousarray(v))


def _golden():
    data = np.load(GOLDEN)
    n = len([k for k in data.files if k.endswith("_op")])
    return [(str(data[f"{i}_op"]), data[f"{i}_A"], data[f"{i}_zi"], data[f"{i}_x"], data[f"{i}_y"],
             str(data[f"{i}_dt"]) if f"{i}_dt" in data.files else "") for i in range(n)]


N_GOLDEN = len([k for k in np.load(GOLDEN).files if k.endswith("_op")])


@pytest.mark.parametrize("case", range(N_GOLDEN))
def test_cpu_op_reproduces_reference_golden_vectors(ops, case):
    """Every golden case bit for bit, half and bfloat16 included (bfloat16
    arrays are stored as their 16-bit patterns)."""
    op, A, zi, x, y, dt = _golden()[case]
    args = [_t(v) for v in (A, zi, x)]
    if dt == "bfloat16":
        args = [v.view(torch.bfloat16) for v in args]
    out = getattr(ops, op)(*args)
    got = (out.view(torch.uint16) if dt == "bfloat16" else out).numpy()
    assert got.dtype == y.dtype and got.shape == y.shape
    np.testing.assert_array_equal(got, y)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 3, 5])
@pytest.mark.parametrize("shared", [False, True])
def test_cpu_recurN_matches_oracle(ops, dtype, M, shared):
    g = D.rng(D.seed_of("cpu-recurN", np.dtype(dtype).str, M, shared))
    B, T = 3, 777
    A = D.stable_matrix(g, (T,) if shared else (B, T), M, dtype)
    zi, x, gy = D.normal(g, (B, M), dtype), D.normal(g, (B, T, M), dtype), D.normal(g, (B, T, M), dtype)
    y = ops.recurN(_t(A), _t(zi), _t(x)).numpy()
    y_ref = oracle.recurN(A, zi, x)
    np.testing.assert_array_equal(y, y_ref)
    if M == 2:
        np.testing.assert_array_equal(ops.recur2(_t(A), _t(zi), _t(x)).numpy(), y_ref)
    gA, gz, gx = (v.numpy() for v in ops.recurN_backward(_t(A), _t(zi), _t(y), _t(gy)))
    rA, rz, rx = oracle.recurN_bwd(A, zi, y_ref, gy)
    np.testing.assert_array_equal(gx, rx)  # the same adjoint recurrence, step for step
    np.testing.assert_array_equal(gz, rz)
    D.check(gA, rA, "grad_A")  # shared A: the same row order; batched: the same products


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("shared", [False, True])
def test_cpu_lti_recurN_matches_oracle(ops, dtype, M, shared):
    g = D.rng(D.seed_of("cpu-lti-recurN", np.dtype(dtype).str, M, shared))
    B, T = 4, 1001
    A = D.stable_matrix(g, () if shared else (B,), M, dtype)
    zi, x, gy = D.normal(g, (B, M), dtype), D.normal(g, (B, T, M), dtype), D.normal(g, (B, T, M), dtype)
    y = ops.lti_recurN(_t(A), _t(zi), _t(x)).numpy()
    y_ref = oracle.lti_recurN(A, zi, x)
    np.testing.assert_array_equal(y, y_ref)
    gA, gz, gx = (v.numpy() for v in ops.lti_recurN_backward(_t(A), _t(zi), _t(y), _t(gy)))
    rA, rz, rx = oracle.lti_recurN_bwd(A, zi, y_ref, gy)
    np.testing.assert_array_equal(gx, rx)
    np.testing.assert_array_equal(gz, rz)
    D.check(gA, rA, "grad_A")  # a sum over time: summed in the other time order here


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("shared", [False, True])
def test_cpu_scalar_ops_match_oracle(ops, dtype, shared):
    g = D.rng(D.seed_of("cpu-scalar", np.dtype(dtype).str, shared))
    B, T = 5, 3001
    zi, x, gy = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype), D.normal(g, (B, T), dtype)
    # LPV: recur
    a = D.coef(g, (T,) if shared else (B, T), dtype)
    y = ops.recur(_t(a), _t(zi), _t(x)).numpy()
    y_ref = oracle.recur(a, zi, x)
    np.testing.assert_array_equal(y, y_ref)
    ga, gz, gx = (v.numpy() for v in ops.recur_backward(_t(a), _t(zi), _t(y), _t(gy)))
    ra, rz, rx = oracle.recur_bwd(a, zi, y_ref, gy)
    np.testing.assert_array_equal(gx, rx)
    np.testing.assert_array_equal(gz, rz)
    D.check(ga, ra, "grad_a")
    # LTI: lti_recur
    c = D.coef(g, (1,) if shared else (B,), dtype)
    y = ops.lti_recur(_t(c), _t(zi), _t(x)).numpy()
    y_ref = oracle.lti_recur(c, zi, x)
    np.testing.assert_array_equal(y, y_ref)
    gc, gz, gx = (v.numpy() for v in ops.lti_recur_backward(_t(c), _t(zi), _t(y), _t(gy)))
    rc, rz, rx = oracle.lti_recur_bwd(c, zi, y_ref, gy)
    D.check(gx, rx, "grad_x")
    D.check(gz, rz, "grad_zi", scale=np.max(np.abs(rx)))
    D.check(gc, rc, "grad_a")


def test_cpu_fibonacci_known_answer(ops):
    """README.md:143-159: lti_recur2 with A = [[1, 1], [1, 0]] and a unit
    impulse gives the Fibonacci numbers, exactly in int64."""
    A = torch.tensor([[1, 1], [1, 0]], dtype=torch.int64)
    x = torch.zeros(1, 10, 2, dtype=torch.int64)
    x[0, 0, 0] = 1
    zi = torch.zeros(1, 2, dtype=torch.int64)
    y = ops.lti_recur2(A, zi, x)
    assert y[0, :, 0].tolist() == [1, 1, 2, 3, 5, 8, 13, 21, 34, 55]


def test_cpu_empty_and_half(ops):
    z = torch.zeros(0, 5)
    assert ops.recur(torch.zeros(0, 5), torch.zeros(0), z).shape == (0, 5)
    gA, gz, gx = ops.recur_backward(torch.zeros(2, 0), torch.ones(2), torch.zeros(2, 0), torch.zeros(2, 0))
    assert gz.tolist() == [0.0, 0.0] and gA.shape == (2, 0)
    g = D.rng(5)
    a = torch.tensor(D.coef(g, (2, 300), np.float32))
    x, zi = torch.randn(2, 300), torch.randn(2)
    for dt in (torch.float16, torch.bfloat16):
        a16, zi16, x16 = a.to(dt), zi.to(dt), x.to(dt)
        y = ops.recur(a16, zi16, x16)
        assert y.dtype == dt
        # the reference's loop in the 16-bit type: every product and sum
        # rounded to it (philtorch/csrc/host_recurN.cpp:81-140 with scalar_t
        # = Half / BFloat16)
        h, ref = zi16.clone(), torch.empty_like(x16)
        for t in range(x16.shape[1]):
            h = x16[:, t] + (torch.zeros_like(h) + a16[:, t] * h)
            ref[:, t] = h
        assert torch.equal(y, ref)
        # backward: the adjoint in the 16-bit type, within its rounding of the fp32 adjoint
        gA, gz, gx = ops.recur_backward(a16, zi16, y, torch.ones_like(y))
        gA32, gz32, gx32 = ops.recur_backward(a16.float(), zi16.float(), y.float(), torch.ones(2, 300))
        for got, want in ((gA, gA32), (gz, gz32), (gx, gx32)):
            assert got.dtype == dt
            assert float((got.float() - want).abs().max()) <= 0.05 * float(want.abs().max())


def test_cpu_errors(ops):
    x = torch.zeros(2, 10)
    with pytest.raises(RuntimeError, match="same scalar type"):
        ops.recur(torch.zeros(2, 10, dtype=torch.float64), torch.zeros(2), x)
    with pytest.raises(RuntimeError, match="A must be a 3D or 4D tensor"):
        ops.recurN(torch.zeros(10, 2), torch.zeros(2, 2), torch.zeros(2, 10, 2))
    with pytest.raises(RuntimeError, match="A must be a vector or a scalar"):
        ops.lti_recur(torch.zeros(2, 2), torch.zeros(2), x)


def test_cpu_opcheck(ops):
    g = D.rng(9)
    B, T = 2, 50
    A2 = torch.tensor(D.stable_matrix(g, (B, T), 2, np.float64))
    L2 = torch.tensor(D.stable_matrix(g, (B,), 3, np.float64))
    zi2, x2 = torch.randn(B, 2, dtype=torch.float64), torch.randn(B, T, 2, dtype=torch.float64)
    zi3, x3 = torch.randn(B, 3, dtype=torch.float64), torch.randn(B, T, 3, dtype=torch.float64)
    a, c = torch.rand(B, T, dtype=torch.float64) - 0.5, torch.rand(B, dtype=torch.float64) - 0.5
    zs, xs = torch.randn(B, dtype=torch.float64), torch.randn(B, T, dtype=torch.float64)
    cases = [
        (ops.recur2.default, (A2, zi2, x2)),
        (ops.recurN.default, (A2, zi2, x2)),
        (ops.lti_recurN.default, (L2, zi3, x3)),
        (ops.lti_recur2.default, (torch.tensor(D.stable_matrix(g, (B,), 2, np.float64)), zi2, x2)),
        (ops.lti_recur.default, (c, zs, xs)),
        (ops.recur.default, (a, zs, xs)),
    ]
    for op, args in cases:
        args = tuple(t.clone().requires_grad_(True) for t in args)
        torch.library.opcheck(op, args)


def test_cpu_api_routes_to_native_ops(ops):
    """The API's indicators send CPU tensors to the native ops, as the
    reference's do, and autograd through them passes gradcheck."""
    from philtorch_amd import lpv, lti
    from philtorch_amd.lpv import ssm as lpv_ssm
    from philtorch_amd.lti import ssm as lti_ssm

    x = torch.zeros(2, 5, dtype=torch.float64)
    assert lpv_ssm.extension_backend_indicator(x, 7)
    assert lti_ssm.extension_backend_indicator(x, 3) and not lti_ssm.extension_backend_indicator(x, 1)
    g = D.rng(11)
    a = torch.tensor(D.coef(g, (2, 40), np.float64), requires_grad=True)
    x = torch.randn(2, 40, dtype=torch.float64, requires_grad=True)
    zi = torch.randn(2, dtype=torch.float64, requires_grad=True)
    torch.autograd.gradcheck(lambda a_, z_, x_: lpv.linear_recurrence(a_, z_, x_, unroll_factor=1), (a, zi, x))
    A = torch.tensor(D.stable_matrix(g, (2, 40), 2, np.float64), requires_grad=True)
    zi2 = torch.randn(2, 2, dtype=torch.float64, requires_grad=True)
    x2 = torch.randn(2, 40, 2, dtype=torch.float64, requires_grad=True)
    torch.autograd.gradcheck(lambda A_, z_, x_: lpv.MatrixRecurrence.apply(A_, z_, x_), (A, zi2, x2))
    p = torch.tensor(D.coef(g, (2,), np.complex128), requires_grad=True)
    zc = torch.randn(2, dtype=torch.complex128, requires_grad=True)
    xc = torch.randn(2, 40, dtype=torch.complex128, requires_grad=True)
    torch.autograd.gradcheck(lambda p_, z_, x_: lti.LTIRecurrence.apply(p_, z_, x_), (p, zc, xc))
