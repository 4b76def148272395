"""Pins of the CPU oracle (CPU only).

The oracle restates philtorch's CPU extension and backward closures; these
tests make sure a plausible slip in that restatement (dropped term, wrong
index or sign, transposed operand) cannot survive:

* golden vectors written by the reference's own CPU operators
  (tests/golden/ref_vectors.npz, from oracle/_ref/ref_C.so built from the
  reference sources) — the forward must match them bit for bit;
* the same comparison live against oracle/_ref when that library is present;
* closed forms: a = 0, a = 1 (cumsum), x = 0 (cumprod), constant a against
  scipy.signal.lfilter;
* an explicit product formula and explicit matrix products on small inputs;
* the README Fibonacci known answer in int64;
* backward: central finite differences (fp64) and the adjoint identity
  <g, J d> = <J^T g, d> with J applied through the (independently pinned)
  forward.
"""
import os

import numpy as np
import pytest
import scipy.signal

import oracle
from tests import _data as D

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")
FLOATS = [np.float32, np.float64, np.complex64, np.complex128]


def _oracle_fwd(op, A, zi, x):
    if op == "recurN":
        return oracle.recurN(A, zi, x)
    if op == "lti_recurN":
        return oracle.lti_recurN(A, zi, x)
    return oracle.lti_recur(A, zi, x)


def _golden_cases():
    """The golden cases in the oracle's dtypes (fp32, fp64, complex, int64);
    the half and bfloat16 cases pin the CPU key only (tests/test_cpu_ops.py):
    the oracle restates the arithmetic of the wider types."""
    data = np.load(GOLDEN)
    n = len([k for k in data.files if k.endswith("_op")])
    return [(str(data[f"{i}_op"]), data[f"{i}_A"], data[f"{i}_zi"], data[f"{i}_x"], data[f"{i}_y"]) for i in range(n)
            if f"{i}_dt" not in data.files and data[f"{i}_A"].dtype != np.float16]


N_GOLDEN = len(_golden_cases())


@pytest.mark.parametrize("case", range(N_GOLDEN))
def test_oracle_matches_reference_golden_vectors(case):
    op, A, zi, x, y = _golden_cases()[case]
    got = _oracle_fwd(op, A, zi, x)
    assert got.dtype == y.dtype and got.shape == y.shape
    np.testing.assert_array_equal(got, y)  # same operations in the same order


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(oracle.__file__), "_ref", "ref_C.so")),
                    reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("dtype", [np.float32, np.complex128])
def test_oracle_matches_live_reference_build(dtype):
    from oracle import ref_runner

    g = D.rng(77)
    B, T = 4, 513
    A = D.biquad_A(g, (B, T), dtype)
    zi, x = D.normal(g, (B, 2), dtype), D.normal(g, (B, T, 2), dtype)
    np.testing.assert_array_equal(oracle.recurN(A, zi, x), ref_runner.run("recurN", A, zi, x))
    a = D.coef(g, (B,), dtype)
    zs, xs = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype)
    np.testing.assert_array_equal(oracle.lti_recur(a, zs, xs), ref_runner.run("lti_recur", a, zs, xs))


# ------------------------------------------------------------ closed forms
@pytest.mark.parametrize("dtype", FLOATS)
def test_closed_forms_scalar(dtype):
    g = D.rng(1)
    B, T = 3, 200
    x, zi = D.normal(g, (B, T), dtype), D.normal(g, (B,), dtype)
    zero, one = np.zeros((B, T), dtype), np.ones((B, T), dtype)
    np.testing.assert_allclose(oracle.recur(zero, zi, x), x)  # a = 0: y = x
    rtol = 1e-4 if np.dtype(dtype) in (np.dtype(np.float32), np.dtype(np.complex64)) else 1e-12
    np.testing.assert_allclose(oracle.recur(one, zi, x), np.cumsum(x, axis=1) + zi[:, None], rtol=rtol, atol=rtol * 20)
    a = D.coef(g, (B, T), dtype)
    np.testing.assert_allclose(oracle.recur(a, zi, np.zeros_like(x)), zi[:, None] * np.cumprod(a, axis=1),
                               rtol=rtol, atol=1e-30)


@pytest.mark.parametrize("dtype", [np.float64, np.complex128])
def test_constant_coefficient_matches_scipy_lfilter(dtype):
    g = D.rng(2)
    B, T = 4, 500
    a = D.coef(g, (B,), dtype)
    x, zi = D.normal(g, (B, T), dtype), D.normal(g, (B,), dtype)
    for b in range(B):
        # y[t] = a y[t-1] + x[t], y[-1] = zi  <=>  lfilter([1], [1, -a], x, zi=[a zi])
        ref, _ = scipy.signal.lfilter([1.0], [1.0, -a[b]], x[b], zi=[a[b] * zi[b]])
        np.testing.assert_allclose(oracle.lti_recur(a, zi, x)[b], ref, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(oracle.recur(np.broadcast_to(a[:, None], (B, T)), zi, x)[b], ref, rtol=1e-12,
                                   atol=1e-12)


def test_explicit_product_formula():
    """y[t] = (prod_{s<=t} a_s) zi + sum_{s<=t} (prod_{s<u<=t} a_u) x_s."""
    g = D.rng(3)
    B, T = 2, 9
    a, x, zi = D.coef(g, (B, T), np.float64), D.normal(g, (B, T), np.float64), D.normal(g, (B,), np.float64)
    ref = np.zeros((B, T))
    for b in range(B):
        for t in range(T):
            acc = np.prod(a[b, : t + 1]) * zi[b]
            for s in range(t + 1):
                acc += np.prod(a[b, s + 1 : t + 1]) * x[b, s]
            ref[b, t] = acc
    np.testing.assert_allclose(oracle.recur(a, zi, x), ref, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("shared", [False, True])
def test_matrix_recursion_explicit_products(shared):
    """h[t] = A[t] h[t-1] + x[t] by explicit numpy matrix-vector products;
    catches a transposed A (row vs column contraction)."""
    g = D.rng(4)
    B, T = 3, 11
    A = g.standard_normal((T, 2, 2) if shared else (B, T, 2, 2)) * 0.7
    x, zi = g.standard_normal((B, T, 2)), g.standard_normal((B, 2))
    ref = np.zeros((B, T, 2))
    for b in range(B):
        h = zi[b]
        for t in range(T):
            h = (A[t] if shared else A[b, t]) @ h + x[b, t]
            ref[b, t] = h
    np.testing.assert_allclose(oracle.recurN(A, zi, x), ref, rtol=1e-13, atol=1e-13)
    # LTI: time-invariant A equals LPV with A repeated along time
    A0 = A[0] if shared else A[:, 0]
    At = np.broadcast_to(A0[..., None, :, :] if not shared else A0, (B, T, 2, 2) if not shared else (T, 2, 2))
    np.testing.assert_allclose(oracle.lti_recurN(A0, zi, x), oracle.recurN(np.ascontiguousarray(At), zi, x),
                               rtol=1e-13, atol=1e-13)


def test_biquad_tdf2_matches_scipy():
    """A transposed-direct-form-II biquad as a 2x2 LTI recursion equals
    scipy.signal.lfilter, with initial state and output y = h[t-1][0] + b0 x."""
    g = D.rng(5)
    T = 400
    b = np.array([0.3, -0.2, 0.5])
    a = np.array([1.0, -1.2, 0.5])
    x = g.standard_normal(T)
    zi = g.standard_normal(2)
    A = np.array([[-a[1], 1.0], [-a[2], 0.0]])  # companion(a)^T
    Bv = b[1:] - b[0] * a[1:]
    h = oracle.lti_recurN(A, zi[None], (x[:, None] * Bv)[None])[0]
    prev = np.vstack([zi[None], h[:-1]])
    y = prev[:, 0] + b[0] * x
    ref, zf = scipy.signal.lfilter(b, a, x, zi=zi)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(h[-1], zf, rtol=1e-12, atol=1e-12)


def test_fibonacci_known_answer():
    """philtorch README.md:143-159: lti_recur2 with [[1,1],[1,0]] in int64."""
    A = np.array([[1, 1], [1, 0]], np.int64)
    x = np.zeros((1, 10, 2), np.int64)
    x[0, 0, 0] = 1
    y = oracle.lti_recurN(A, np.zeros((1, 2), np.int64), x)
    assert y[0, :, 0].tolist() == [1, 1, 2, 3, 5, 8, 13, 21, 34, 55]


# ------------------------------------------------------------ backward
def _fd_grad(f, v, eps=1e-6):
    """Central differences of the scalar f(v) for real v (fp64)."""
    g = np.zeros_like(v)
    it = np.nditer(v, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        vp, vm = v.copy(), v.copy()
        vp[i] += eps
        vm[i] -= eps
        g[i] = (f(vp) - f(vm)) / (2 * eps)
    return g


@pytest.mark.parametrize("kind", ["recur", "recur_shared", "lti", "lti_shared", "recurN", "recurN_shared",
                                  "lti_recurN", "lti_recurN_shared", "recurN3", "recurN4_shared", "lti_recurN3_shared",
                                  "lti_recurN4"])
def test_backward_finite_differences(kind):
    g = D.rng(D.seed_of("fd", kind))
    B, T = 2, 6
    base = kind.replace("_shared", "")
    M = int(base[-1]) if base[-1].isdigit() else 2  # matrix order of the recurN / lti_recurN kinds
    if kind.startswith("recurN"):
        A = g.standard_normal((T, M, M) if kind.endswith("shared") else (B, T, M, M)) * 0.6 / M ** 0.5
        zi, x, gy = g.standard_normal((B, M)), g.standard_normal((B, T, M)), g.standard_normal((B, T, M))
        fwd, bwd = oracle.recurN, oracle.recurN_bwd
    elif kind.startswith("lti_recurN"):
        A = g.standard_normal((M, M) if kind.endswith("shared") else (B, M, M)) * 0.6 / M ** 0.5
        zi, x, gy = g.standard_normal((B, M)), g.standard_normal((B, T, M)), g.standard_normal((B, T, M))
        fwd, bwd = oracle.lti_recurN, oracle.lti_recurN_bwd
    elif kind.startswith("lti"):
        A = g.uniform(-0.9, 0.9, (1,) if kind.endswith("shared") else (B,))
        zi, x, gy = g.standard_normal(B), g.standard_normal((B, T)), g.standard_normal((B, T))
        fwd, bwd = oracle.lti_recur, oracle.lti_recur_bwd
    else:
        A = g.uniform(-0.9, 0.9, (T,) if kind.endswith("shared") else (B, T))
        zi, x, gy = g.standard_normal(B), g.standard_normal((B, T)), g.standard_normal((B, T))
        fwd, bwd = oracle.recur, oracle.recur_bwd
    y = fwd(A, zi, x)
    gA, gzi, gx = bwd(A, zi, y, gy)
    loss = lambda A_, zi_, x_: float(np.sum(fwd(A_, zi_, x_) * gy))  # noqa: E731
    np.testing.assert_allclose(gA, _fd_grad(lambda v: loss(v, zi, x), A).reshape(gA.shape), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gzi, _fd_grad(lambda v: loss(A, v, x), zi), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gx, _fd_grad(lambda v: loss(A, zi, v), x), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [np.float64, np.complex128])
def test_backward_adjoint_identity(dtype):
    """For fixed A the forward is linear in (zi, x): J d = recur(A, dzi, dx).
    Then <g, J d> must equal <grad_zi, dzi> + <grad_x, dx> (real inner
    products; complex uses Re<u, v> with the conjugate-linear convention)."""
    g = D.rng(6)
    B, T = 3, 300
    A = D.coef(g, (B, T), dtype)
    zi, x, gy = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype), D.normal(g, (B, T), dtype)
    dzi, dx = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype)
    y = oracle.recur(A, zi, x)
    _, gzi, gx = oracle.recur_bwd(A, zi, y, gy)
    Jd = oracle.recur(A, dzi, dx)
    lhs = np.real(np.vdot(gy, Jd))
    rhs = np.real(np.vdot(gzi, dzi)) + np.real(np.vdot(gx, dx))
    assert abs(lhs - rhs) <= 1e-10 * max(1.0, abs(lhs))


def test_complex_coefficient_gradient_convention():
    """grad_A = lambda conj(h[t-1]): the Wirtinger convention torch uses for
    complex autograd; checked against torch.autograd on a tiny fp64 loop."""
    import torch

    g = D.rng(7)
    B, T = 2, 5
    A = D.coef(g, (B, T), np.complex128)
    zi, x, gy = D.normal(g, (B,), np.complex128), D.normal(g, (B, T), np.complex128), D.normal(g, (B, T), np.complex128)
    tA = torch.tensor(A, requires_grad=True)
    h = torch.tensor(zi)
    outs = []
    for t in range(T):
        h = tA[:, t] * h + torch.tensor(x[:, t])
        outs.append(h)
    torch.stack(outs, 1).backward(torch.tensor(gy))
    y = oracle.recur(A, zi, x)
    gA, _, _ = oracle.recur_bwd(A, zi, y, gy)
    np.testing.assert_allclose(gA, tA.grad.numpy(), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- SOS cascade
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("batched", [False, True])
def test_sosfilt_matches_scipy(dtype, batched):
    """oracle.sosfilt (one lfilter(tdf2) per section through the oracle's
    lti_recurN) against scipy.signal.sosfilt, with initial states."""
    g = D.rng(D.seed_of("oracle-sos", dtype, batched))
    B, T, S = 3, 700, 5
    sos = D.sos_coefs(g, (B,) if batched else (), S, np.float64)
    x = g.standard_normal((B, T))
    zi = g.standard_normal((B, S, 2))
    y, zf = oracle.sosfilt(sos.astype(dtype), x.astype(dtype), zi.astype(dtype))
    for b in range(B):
        ry, rzf = scipy.signal.sosfilt(sos[b] if batched else sos, x[b], zi=zi[b])
        D.check(y[b], ry.astype(dtype), f"y row {b}")
        # zf on the signal's scale: fp32 arithmetic (the reference's own) leaves
        # ~1e-5 of max|y| on the final states of the later sections
        err = np.max(np.abs(zf[b] - rzf))
        assert err <= D.tol(dtype) * max(np.max(np.abs(ry)), np.max(np.abs(rzf))), f"zf row {b}: {err}"


def _sos_serial_loop(sos, x, zi):
    """The TDF-II difference equations of each section, written step by step
    in torch (y = b0 u + z1; z1 = b1 u - a1 y + z2; z2 = b2 u - a2 y), so that
    autograd derives the cascade's gradient independently of the oracle."""
    import torch

    u, zfs = x, []
    for s in range(sos.shape[-2]):
        b0, b1, b2, a1, a2 = (sos[..., s, i] for i in (0, 1, 2, 4, 5))
        z1, z2 = zi[:, s, 0], zi[:, s, 1]
        ys = []
        for t in range(x.shape[1]):
            yt = b0 * u[:, t] + z1
            z1, z2 = b1 * u[:, t] - a1 * yt + z2, b2 * u[:, t] - a2 * yt
            ys.append(yt)
        u = torch.stack(ys, 1)
        zfs.append(torch.stack([z1, z2], -1))
    return u, torch.stack(zfs, 1)


@pytest.mark.parametrize("batched", [False, True])
def test_sosfilt_backward_matches_serial_autograd(batched):
    import torch

    g = D.rng(D.seed_of("oracle-sos-bwd", batched))
    B, T, S = 3, 30, 4
    sos = D.sos_coefs(g, (B,) if batched else (), S, np.float64)
    x = g.standard_normal((B, T))
    zi = g.standard_normal((B, S, 2))
    gy = g.standard_normal((B, T))
    gzf = g.standard_normal((B, S, 2))
    ts, tx, tz = (torch.tensor(v, requires_grad=True) for v in (sos, x, zi))
    y, zf = _sos_serial_loop(ts, tx, tz)
    ((y * torch.tensor(gy)).sum() + (zf * torch.tensor(gzf)).sum()).backward()
    gs, gzi, gx = oracle.sosfilt_bwd(sos, x, zi, gy, gzf)
    ref_gs = ts.grad.numpy().copy()
    ref_gs[..., 3] = 0  # a0 appears in no difference equation
    D.check(gs, ref_gs, "grad_sos")
    D.check(gzi, tz.grad.numpy(), "grad_zi")
    D.check(gx, tx.grad.numpy(), "grad_x")


# ---------------------------------------------------------------- filtfilt
def _scipy_filtfilt_composed(b, a, x, np_mode, edge):
    """filtfilt step by step on scipy's lfilter_zi and lfilter, with numpy's
    padding (for the pad modes scipy.signal.filtfilt has no padtype for)."""
    den = np.r_[1.0, a]
    ext = np.pad(x, (edge, edge), mode=np_mode) if edge else x
    zi = scipy.signal.lfilter_zi(b, den)
    y, _ = scipy.signal.lfilter(b, den, ext, zi=zi * ext[0])
    y2, _ = scipy.signal.lfilter(b, den, y[::-1], zi=zi * y[-1])
    return (y2[edge:-edge] if edge else y2)[::-1]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("batched", [False, True])
def test_filtfilt_matches_scipy(dtype, batched):
    """oracle.filtfilt against scipy.signal.filtfilt: F.pad's "replicate" is
    scipy's padtype "constant" (edge values), "reflect" is "even", and no
    padding is padtype None; "constant" (zeros) and "circular" against the
    same steps on scipy's lfilter_zi / lfilter and numpy's padding."""
    g = D.rng(D.seed_of("oracle-filtfilt", dtype, batched))
    B, T = 3, 500
    sos = D.sos_coefs(g, (B,) if batched else (), 1, np.float64, rhi=0.98)[..., 0, :]
    x = g.standard_normal((B, T))
    cases = [("replicate", 9, "constant"), ("reflect", 9, "even"), ("replicate", 40, "constant"),
             ("reflect", T - 1, "even"), (None, None, None)]
    for padmode, padlen, padtype in cases:
        y = oracle.filtfilt(sos.astype(dtype), x.astype(dtype), padmode=padmode, padlen=padlen)
        for r in range(B):
            s = sos[r] if batched else sos
            ref = scipy.signal.filtfilt(s[:3], np.r_[1.0, s[4:]], x[r], padtype=padtype,
                                        padlen=padlen if padtype else None)
            D.check(y[r], ref.astype(dtype), f"{padmode} {padlen} row {r}")
    for padmode, np_mode in (("constant", "constant"), ("circular", "wrap")):
        for padlen in (9, T - 1):
            y = oracle.filtfilt(sos.astype(dtype), x.astype(dtype), padmode=padmode, padlen=padlen)
            for r in range(B):
                s = sos[r] if batched else sos
                ref = _scipy_filtfilt_composed(s[:3], s[4:], x[r], np_mode, padlen)
                D.check(y[r], ref.astype(dtype), f"{padmode} {padlen} row {r}")


def test_filtfilt_steady_state_and_lfilter_zi():
    """A constant row comes out scaled by H(1)^2 for every edge-value pad (the
    padded row is constant and both passes start in their steady state), and
    lfilter_zi is the fixed point of one TDF-II step."""
    g = D.rng(D.seed_of("oracle-filtfilt-dc"))
    sos = D.sos_coefs(g, (4,), 1, np.float64)[:, 0, :]
    h1 = sos[:, :3].sum(-1) / (1 + sos[:, 4] + sos[:, 5])
    x = np.full((4, 300), 2.5)
    for padmode in ("replicate", "reflect", "circular", None):
        y = oracle.filtfilt(sos, x, padmode=padmode)
        np.testing.assert_allclose(y, (h1 * h1 * 2.5)[:, None] * np.ones((1, 300)), rtol=1e-12)
    zi = oracle.lfilter_zi(sos)
    A, Bv, _, _ = oracle._tdf2_section(sos)
    np.testing.assert_allclose(np.einsum("rij,rj->ri", A, zi) + Bv, zi, rtol=1e-12)


@pytest.mark.parametrize("order", [1, 2, 3, 4])
@pytest.mark.parametrize("batched", [False, True])
def test_filtfilt_ba_matches_scipy(order, batched):
    """oracle.filtfilt_ba (any order, the TDF-II companion model through
    lti_state_space) against scipy.signal.filtfilt for the edge-value pads
    and no padding, and against the same steps on scipy's lfilter_zi /
    lfilter for zeros and circular padding; its default pad length is
    3 * max(nb, na + 1), as the reference's."""
    g = D.rng(D.seed_of("oracle-filtfilt-ba", order, batched))
    B, T = 3, 400
    b, a = D.ba_coefs(g, (B,) if batched else (), order, np.float64, rhi=0.97)
    x = g.standard_normal((B, T))
    ntaps = order + 1
    for padmode, padlen, padtype in (("replicate", None, "constant"), ("reflect", 25, "even"),
                                     ("replicate", T - 1, "constant"), (None, None, None)):
        y = oracle.filtfilt_ba(b, a, x, padmode=padmode, padlen=padlen)
        for r in range(B):
            br, ar = (b[r], a[r]) if batched else (b, a)
            pl = (3 * ntaps if padlen is None else padlen) if padtype else None
            ref = scipy.signal.filtfilt(br, np.r_[1.0, ar], x[r], padtype=padtype, padlen=pl)
            D.check(y[r], ref, f"order {order} {padmode} {padlen} row {r}")
    for padmode, np_mode in (("constant", "constant"), ("circular", "wrap")):
        for padlen in (7, T - 1):
            y = oracle.filtfilt_ba(b, a, x, padmode=padmode, padlen=padlen)
            for r in range(B):
                br, ar = (b[r], a[r]) if batched else (b, a)
                ref = _scipy_filtfilt_composed(br, ar, x[r], np_mode, padlen)
                D.check(y[r], ref, f"order {order} {padmode} {padlen} row {r}")


def test_filtfilt_ba_agrees_with_biquad_oracle_and_steady_state():
    """filtfilt_ba of a biquad is oracle.filtfilt of its section (the cascade
    route); lfilter_zi_ba is the fixed point of one TDF-II step at every
    order; a constant row comes out scaled by H(1)^2."""
    g = D.rng(D.seed_of("oracle-filtfilt-ba-x"))
    sos = D.sos_coefs(g, (3,), 1, np.float64)[:, 0, :]
    x = g.standard_normal((3, 300))
    for padmode in ("replicate", "reflect", "constant", "circular", None):
        D.check(oracle.filtfilt_ba(sos[:, :3], sos[:, 4:], x, padmode=padmode),
                oracle.filtfilt(sos, x, padmode=padmode), f"biquad {padmode}")
    for order in (1, 2, 3, 4):
        b, a = D.ba_coefs(g, (4,), order, np.float64)
        A, gv, _ = oracle._tdf2_companion(b, a)
        zi = oracle.lfilter_zi_ba(b, a)
        np.testing.assert_allclose(np.einsum("rij,rj->ri", A, zi) + gv, zi, rtol=1e-12, atol=1e-12)
        h1 = b.sum(-1) / (1 + a.sum(-1))
        for padmode in ("replicate", "reflect", "circular"):
            y = oracle.filtfilt_ba(b, a, np.full((4, 200), -1.5), padmode=padmode)
            np.testing.assert_allclose(y, np.broadcast_to((h1 * h1 * -1.5)[:, None], (4, 200)), rtol=1e-10)


# ---------------------------------------------------------------- SISO state space
def _stable_model(g, M, lead=()):
    """A dense A with a stable spectrum (a companion matrix of poles of radius
    < 0.97, conjugated by a well-conditioned random basis), B, C, D."""
    shape = tuple(lead)
    r = g.uniform(0.3, 0.97, shape + (M,))
    th = g.uniform(0, np.pi, shape + (M,))
    poles = r * np.exp(1j * th)
    poles[..., 1::2] = np.conj(poles[..., 0::2][..., : M // 2])
    if M % 2:
        poles[..., -1] = r[..., -1] * np.sign(g.uniform(-1, 1, shape))
    a = np.real(np.apply_along_axis(np.poly, -1, poles.reshape(-1, M)).reshape(shape + (M + 1,)))[..., 1:]
    comp = np.zeros(shape + (M, M))
    comp[..., 0, :] = -a
    comp[..., np.arange(1, M), np.arange(M - 1)] = 1.0
    V = np.eye(M) + 0.3 * g.standard_normal(shape + (M, M))
    A = V @ comp @ np.linalg.inv(V)
    return A, g.standard_normal(shape + (M,)), g.standard_normal(shape + (M,)), g.standard_normal(shape)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_lti_state_space_matches_scipy_dlsim(M):
    """oracle.lti_state_space (B x, lti_recurN, shift, C h + D x) against
    scipy.signal.dlsim (x[k+1] = A x[k] + B u[k], y[k] = C x[k] + D u[k]), per
    row, with initial states; and its B = None / out_idx forms."""
    g = D.rng(D.seed_of("oracle-ss", M))
    Bn, T = 3, 400
    A, Bv, Cv, Dv = _stable_model(g, M, (Bn,))
    x = g.standard_normal((Bn, T))
    zi = g.standard_normal((Bn, M))
    y, zf = oracle.lti_state_space(A, x, Bv, Cv, Dv, zi)
    for r in range(Bn):
        _, ry, rx = scipy.signal.dlsim((A[r], Bv[r][:, None], Cv[r][None, :], [[Dv[r]]], 1), x[r], x0=zi[r])
        D.check(y[r], ry[:, 0], f"y row {r}")
        rzf = A[r] @ rx[-1] + Bv[r] * x[r, -1]
        D.check(zf[r], rzf, f"zf row {r}", scale=np.max(np.abs(ry)))
    e0 = np.eye(M)[0]
    idx = M - 1
    y2, _ = oracle.lti_state_space(A[0], x, None, None, None, zi, out_idx=idx)
    for r in range(Bn):
        _, ry, _ = scipy.signal.dlsim((A[0], e0[:, None], np.eye(M)[idx][None, :], [[0.0]], 1), x[r], x0=zi[r])
        D.check(y2[r], ry[:, 0], f"out_idx row {r}")


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("F,P", [(1, 1), (2, 3), (4, 4), (3, 1)])
def test_lti_state_space_mimo_matches_scipy_dlsim(M, F, P):
    """oracle.lti_state_space_mimo (B x per step, lti_recurN, shift, C h + D x)
    against scipy.signal.dlsim's multi-input multi-output simulation, per row,
    with per-row and shared operands and initial states: a transposed B, C or
    D, or a state shift off by one, fails it."""
    g = D.rng(D.seed_of("oracle-ss-mimo", M, F, P))
    Bn, T = 3, 300
    A, _, _, _ = _stable_model(g, M, (Bn,))
    Bm, Cm, Dm = g.standard_normal((Bn, M, F)), g.standard_normal((P, M)), g.standard_normal((Bn, P, F))
    x = g.standard_normal((Bn, T, F))
    zi = g.standard_normal((Bn, M))
    y, zf = oracle.lti_state_space_mimo(A, x, Bm, Cm, Dm, zi)
    assert y.shape == (Bn, T, P) and zf.shape == (Bn, M)
    for r in range(Bn):
        _, ry, rx = scipy.signal.dlsim((A[r], Bm[r], Cm, Dm[r], 1), x[r], x0=zi[r])
        D.check(y[r], ry.reshape(T, P), f"y row {r}")
        D.check(zf[r], A[r] @ rx[-1] + Bm[r] @ x[r, -1], f"zf row {r}", scale=np.max(np.abs(ry)))
    # shared A and B, no D, no zi: the zero-state response
    y2, _ = oracle.lti_state_space_mimo(A[0], x, Bm[0], Cm)
    for r in range(Bn):
        _, ry, _ = scipy.signal.dlsim((A[0], Bm[0], Cm, np.zeros((P, F)), 1), x[r])
        D.check(y2[r], ry.reshape(T, P), f"shared row {r}")


def test_lti_state_space_mimo_reduces_to_siso():
    """With one input and one output the matrix form is the single-input
    single-output oracle (pinned to dlsim above) on the same operands; and an
    empty row returns zi as its final state."""
    g = D.rng(D.seed_of("oracle-ss-mimo-siso"))
    Bn, T, M = 2, 90, 3
    A, Bv, Cv, Dv = _stable_model(g, M, (Bn,))
    x = g.standard_normal((Bn, T))
    zi = g.standard_normal((Bn, M))
    y1, zf1 = oracle.lti_state_space(A, x, Bv, Cv, Dv, zi)
    y2, zf2 = oracle.lti_state_space_mimo(A, x[..., None], Bv[..., None], Cv[:, None, :], Dv[:, None, None], zi)
    np.testing.assert_allclose(y2[..., 0], y1, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(zf2, zf1, rtol=1e-12, atol=1e-12)
    y0, zf0 = oracle.lti_state_space_mimo(A, np.zeros((Bn, 0, 2)), np.ones((M, 2)), np.ones((1, M)), None, zi)
    assert y0.shape == (Bn, 0, 1)
    np.testing.assert_array_equal(zf0, zi)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_lpv_state_space_mimo_matches_loop_and_lti(M):
    """oracle.lpv_state_space_mimo against the textbook per-step loop of
    h[t+1] = A[t] h[t] + B x[t], y[t] = C h[t] + D x[t] (per-row and shared
    operands, 2 inputs and 3 outputs), against lti_state_space_mimo (pinned
    to dlsim) when A does not vary along time, and against the
    single-input single-output LPV oracle at F = P = 1."""
    g = D.rng(D.seed_of("oracle-lpv-mimo", M))
    Bn, T, F, P = 3, 50, 2, 3
    A = 0.6 * g.standard_normal((Bn, T, M, M)) / np.sqrt(M)
    Bm, Cm, Dm = g.standard_normal((M, F)), g.standard_normal((Bn, P, M)), g.standard_normal((P, F))
    x = g.standard_normal((Bn, T, F))
    zi = g.standard_normal((Bn, M))
    y, zf = oracle.lpv_state_space_mimo(A, x, Bm, Cm, Dm, zi)
    for r in range(Bn):
        h = zi[r].copy()
        for t in range(T):
            ref = Cm[r] @ h + Dm @ x[r, t]
            np.testing.assert_allclose(y[r, t], ref, rtol=1e-12, atol=1e-12)
            h = A[r, t] @ h + Bm @ x[r, t]
        np.testing.assert_allclose(zf[r], h, rtol=1e-12, atol=1e-12)
    A0 = A[:, 0]
    yl, zl = oracle.lpv_state_space_mimo(np.broadcast_to(A0[:, None], (Bn, T, M, M)), x, Bm, Cm, Dm, zi)
    ym, zm = oracle.lti_state_space_mimo(A0, x, Bm, Cm, Dm, zi)
    np.testing.assert_allclose(yl, ym, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(zl, zm, rtol=1e-12, atol=1e-12)
    ys, zs = oracle.lpv_state_space(A, x[..., 0], Bm[:, 0], Cm[:, 0][:, None, :], Dm[0, 0], zi)
    y1, z1 = oracle.lpv_state_space_mimo(A, x[..., :1], Bm[:, :1], Cm[:, :1], Dm[:1, :1], zi)
    np.testing.assert_allclose(y1[..., 0], ys, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(z1, zs, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- LPV SISO state space
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_lpv_state_space_matches_loop_and_lti(M):
    """oracle.lpv_state_space against the textbook per-step loop of
    h[t+1] = A[t] h[t] + b[t] x[t], y[t] = c[t] . h[t] + d[t] x[t] (per-row
    and per-step operands, shared ones, B / C absent), and against
    lti_state_space when A, b, c, d do not vary along time."""
    g = D.rng(D.seed_of("oracle-lpv-ss", M))
    Bn, T = 3, 60
    A = 0.6 * g.standard_normal((Bn, T, M, M)) / np.sqrt(M)
    x = g.standard_normal((Bn, T))
    zi = g.standard_normal((Bn, M))
    Bv, Cv, Dv = g.standard_normal((Bn, T, M)), g.standard_normal((1, T, M)), g.standard_normal((Bn, 1))
    y, zf = oracle.lpv_state_space(A, x, Bv, Cv, Dv, zi)
    for r in range(Bn):
        h = zi[r].copy()
        for t in range(T):
            ref = Cv[0, t] @ h + Dv[r, 0] * x[r, t]
            assert abs(y[r, t] - ref) <= 1e-12 * (1 + abs(ref))
            h = A[r, t] @ h + Bv[r, t] * x[r, t]
        np.testing.assert_allclose(zf[r], h, rtol=1e-12, atol=1e-12)
    y2, _ = oracle.lpv_state_space(A, x, None, None, None, zi, out_idx=M - 1)
    for r in range(Bn):
        h = zi[r].copy()
        for t in range(T):
            assert abs(y2[r, t] - h[M - 1]) <= 1e-12 * (1 + abs(h[M - 1]))
            e = np.zeros(M)
            e[0] = x[r, t]
            h = A[r, t] @ h + e
    A0, b0, c0, d0 = _stable_model(g, M, (Bn,))
    yl, zl = oracle.lpv_state_space(np.broadcast_to(A0[:, None], (Bn, T, M, M)), x, b0[:, None], c0[:, None],
                                    d0[:, None], zi)
    yr, zr = oracle.lti_state_space(A0, x, b0, c0, d0, zi)
    D.check(yl, yr, "lpv vs lti y")
    D.check(zl, zr, "lpv vs lti zf")
