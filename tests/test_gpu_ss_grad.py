"""GPU parity of the fused coefficient gradients of the single-input
single-output LTI state space and of lfilter (phs_lti_ss_bwd /
philtorch::lti_ss_backward, phs_lfilter_bwd / philtorch::lfilter_ss_backward).

Pins:

* directional derivatives of the oracle (oracle.lti_state_space, pinned to
  scipy.signal.dlsim in tests/test_oracle.py): for a random direction V of
  each input, grad . V against the central difference of
  L = <g, y> + <g_zf, zf> evaluated by the oracle in fp64 (L is linear in
  each of b, c, d, zi and x, so their differences are exact for any step and
  are taken with a large one; A's with a small one) -- a dropped term, a
  transposed A or a wrong index in any gradient fails it;
* the autograd of the composed route the fused kernels replace (B x, the
  native scan, the state shift, C h + D x; philtorch/lti/ssm.py:386-589 and
  lti/filtering.py:273-333), on the same inputs, fp32 and fp64, every operand
  layout, orders 1-4, forward and reversed calls, rows of one step, a tile
  (6144 fp32 / 3072 fp64 steps) and around it, and many tiles;
* the API: lti.state_space and lti.lfilter keep the fused route when a
  coefficient needs a gradient, and gradcheck passes through it.
"""
import numpy as np
import pytest

import oracle
from tests import _data as D
from tests.test_oracle import _stable_model

pytestmark = pytest.mark.gpu

FLOATS = [np.float32, np.float64]
ORDERS = [1, 2, 3, 4]
# (A per row, b, c, d): None absent, "s" shared, "r" per row
LAYOUTS = [(True, "r", "r", "r"), (False, "s", "s", "s"), (True, None, None, None), (False, "r", None, "r"),
           (True, "s", "r", None), (False, None, "s", "s")]


def _normal_model(g, M, lead):
    """A normal A of spectral norm < 0.97 (scaled 2x2 rotations and a real
    pole, in a random orthogonal basis): no transient growth, so fp32
    rounding stays at its own level over long rows."""
    A = np.zeros(tuple(lead) + (M, M))
    for i in range(0, M - 1, 2):
        r, th = g.uniform(0.5, 0.97, lead), g.uniform(0, np.pi, lead)
        A[..., i, i], A[..., i, i + 1] = r * np.cos(th), -r * np.sin(th)
        A[..., i + 1, i], A[..., i + 1, i + 1] = r * np.sin(th), r * np.cos(th)
    if M % 2:
        A[..., M - 1, M - 1] = g.uniform(-0.97, 0.97, lead)
    Q, _ = np.linalg.qr(g.standard_normal((M, M)))
    return Q @ A @ Q.T


def _operands(g, M, Bn, T, layout, dtype, normal=False):
    """normal: a normal A (the fp32 comparisons); otherwise a dense
    non-normal one (a companion matrix in a random basis)."""
    A_row, kb, kc, kd = layout
    lead = (Bn,) if A_row else ()
    A = _normal_model(g, M, lead) if normal else _stable_model(g, M, lead)[0]
    vec = lambda k: None if k is None else g.standard_normal((M,) if k == "s" else (Bn, M))  # noqa: E731
    b, c = vec(kb), vec(kc)
    d = None if kd is None else g.standard_normal((1,) if kd == "s" else (Bn,))
    zi = g.standard_normal((Bn, M))
    x = g.standard_normal((Bn, T))
    cast = lambda v: None if v is None else np.ascontiguousarray(v, dtype=dtype)  # noqa: E731
    return [cast(v) for v in (A, b, c, d, zi, x)]


def _t(v, dev="cuda", rg=False):
    import torch

    return None if v is None else torch.tensor(v, device=dev, requires_grad=rg)


def _oracle_loss(ops, gy, gzf, out_idx, rev):
    A, b, c, d, zi, x = ops
    xs = np.ascontiguousarray(x[:, ::-1]) if rev else x
    y, zf = oracle.lti_state_space(A, xs, b, c, d, zi, out_idx=None if c is not None else out_idx)
    if rev:
        y = y[:, ::-1]
    return float(np.sum(gy * y) + np.sum(gzf * zf))


@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: "".join(str(v)[0] for v in l))
@pytest.mark.parametrize("rev", [False, True])
def test_lti_ss_backward_directional_derivative_vs_oracle(hip, M, layout, rev):
    import torch

    g = D.rng(D.seed_of("ss-grad-fd", M, layout, rev))
    Bn, T = 3, 7001  # fp64 tiles of 3072 steps: three per row, the last ragged
    ops = _operands(g, M, Bn, T, layout, np.float64)
    out_idx = M - 1
    gy, gzf = g.standard_normal((Bn, T)), g.standard_normal((Bn, M))
    print(f"lti_ss_backward fd M={M} layout={layout} rev={rev}", flush=True)
    res = torch.ops.philtorch.lti_ss_backward(*[_t(v) for v in ops], _t(gy), _t(gzf), out_idx, rev)
    grads = [r.cpu().numpy() for r in res]  # gA, gb, gc, gd, gzi, gx
    V = [None if v is None else g.standard_normal(v.shape) for v in ops]
    for i in range(6):
        if ops[i] is None:
            continue
        eps, rtol = (1e-6, 1e-5) if i == 0 else (1.0, 1e-7)
        p = [v if j != i else v + eps * V[i] for j, v in enumerate(ops)]
        m = [v if j != i else v - eps * V[i] for j, v in enumerate(ops)]
        fdi = (_oracle_loss(p, gy, gzf, out_idx, rev) - _oracle_loss(m, gy, gzf, out_idx, rev)) / (2 * eps)
        pi = float(np.sum(grads[i] * V[i]))
        assert abs(pi - fdi) <= rtol * max(1.0, abs(fdi)), (i, pi, fdi)


def _composite_grads(ops, gy, gzf, out_idx, rev, dev):
    """Autograd of the composed route on `dev` (fp64 reference)."""
    import torch

    from philtorch_amd.lti.ssm import _state_space_composite

    ts = [_t(v, dev, v is not None) for v in ops]
    A, b, c, d, zi, x = ts
    xs = x.flip(-1) if rev else x
    y, zf = _state_space_composite(A, b, c, d, zi, xs, out_idx=None if c is not None else out_idx)
    if rev:
        y = y.flip(-1)
    loss = (y * _t(gy, dev)).sum() + (zf * _t(gzf, dev)).sum()
    wrt = [t for t in ts if t is not None]
    gr = torch.autograd.grad(loss, wrt)
    out, k = [], 0
    for t in ts:
        out.append(None if t is None else gr[k].cpu().numpy())
        k += t is not None
    return out


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("Bn,T", [(2, 1), (3, 777), (2, 3072), (2, 6144), (3, 6145), (2, 40001)])
def test_lti_ss_backward_vs_composed_route(hip, dtype, M, Bn, T):
    import torch

    for li, layout in enumerate(LAYOUTS):
        for rev in (False, True):
            g = D.rng(D.seed_of("ss-grad-comp", np.dtype(dtype).str, M, Bn, T, li, rev))
            ops = _operands(g, M, Bn, T, layout, dtype, normal=dtype == np.float32)
            out_idx = 0 if M == 1 else 1
            gy = g.standard_normal((Bn, T)).astype(dtype)
            gzf = g.standard_normal((Bn, M)).astype(dtype)
            print(f"lti_ss_backward {np.dtype(dtype).name} M={M} B={Bn} T={T} layout={layout} rev={rev}", flush=True)
            res = torch.ops.philtorch.lti_ss_backward(*[_t(v) for v in ops], _t(gy), _t(gzf), out_idx, rev)
            got = [r.cpu().numpy() for r in res]
            # the forward keeping its states (phs_lti_ss_fwd_hs; other tile lengths, so y within
            # tolerance of lti_ss's) and the backward given them: the same gradients, bit for bit
            y1, zf1 = torch.ops.philtorch.lti_ss(*[_t(v) for v in ops], out_idx, rev)
            y2, zf2, hs = torch.ops.philtorch.lti_ss_states(*[_t(v) for v in ops], out_idx, rev)
            assert hs.shape == (Bn, T, M)
            D.check(y2.cpu().numpy(), y1.cpu().numpy(), "lti_ss_states y", dtype=dtype)
            D.check(zf2.cpu().numpy(), zf1.cpu().numpy(), "lti_ss_states zf", dtype=dtype)
            res_hs = torch.ops.philtorch.lti_ss_backward(*[_t(v) for v in ops], _t(gy), _t(gzf), out_idx, rev, hs)
            for r0, r1 in zip(res, res_hs):
                assert torch.equal(r0, r1)
            ref = _composite_grads([None if v is None else v.astype(np.float64) for v in ops],
                                   gy.astype(np.float64), gzf.astype(np.float64), out_idx, rev, "cpu")
            names = ("grad_A", "grad_B", "grad_C", "grad_D", "grad_zi", "grad_x")
            for i, nm in enumerate(names):
                if ops[i] is None:
                    assert got[i].size == 0
                    continue
                D.check(got[i], ref[i], f"{nm} layout={layout} rev={rev}", dtype=dtype)


def _lfilter_operands(g, nb, na, Bn, T, shared, dtype):
    """Stable denominators (poles of radius < 0.95), random numerators."""
    lead = () if shared else (Bn,)
    r = g.uniform(0.3, 0.95, lead + (na,))
    th = g.uniform(0, np.pi, lead + (na,))
    p = r * np.exp(1j * th)
    p[..., 1::2] = np.conj(p[..., 0::2][..., : na // 2])
    if na % 2:
        p[..., -1] = r[..., -1]
    a = np.real(np.apply_along_axis(np.poly, -1, p.reshape(-1, na)).reshape(lead + (na + 1,)))[..., 1:]
    b = g.standard_normal(lead + (nb,))
    M = max(nb - 1, na)
    zi = g.standard_normal((Bn, M))
    x = g.standard_normal((Bn, T))
    return [np.ascontiguousarray(v, dtype=dtype) for v in (b, a, zi, x)]


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("nb,na", [(1, 1), (2, 1), (3, 2), (2, 3), (5, 4), (3, 4), (5, 2), (4, 3)])
@pytest.mark.parametrize("form", [0, 1], ids=["tdf2", "df2"])
@pytest.mark.parametrize("shared", [False, True])
def test_lfilter_ss_backward_vs_composed_route(hip, dtype, nb, na, form, shared):
    import torch

    from philtorch_amd.lti.filtering import _ssm_lfilter

    Bn, T = 3, 13001
    for rev in (False, True):
        g = D.rng(D.seed_of("lfilter-grad", np.dtype(dtype).str, nb, na, form, shared, rev))
        b, a, zi, x = _lfilter_operands(g, nb, na, Bn, T, shared, dtype)
        M = zi.shape[1]
        gy, gzf = g.standard_normal((Bn, T)).astype(dtype), g.standard_normal((Bn, M)).astype(dtype)
        print(f"lfilter_ss_backward {np.dtype(dtype).name} nb={nb} na={na} form={form} shared={shared} rev={rev}",
              flush=True)
        res = torch.ops.philtorch.lfilter_ss_backward(_t(b), _t(a), _t(zi), _t(x), _t(gy), _t(gzf), form, rev)
        got = [r.cpu().numpy() for r in res]
        # the states-keeping forward, and the backward given its states: bit for bit
        y1, zf1 = torch.ops.philtorch.lfilter_ss(_t(b), _t(a), _t(zi), _t(x), form, rev)
        y2, zf2, hs = torch.ops.philtorch.lfilter_ss_states(_t(b), _t(a), _t(zi), _t(x), form, rev)
        D.check(y2.cpu().numpy(), y1.cpu().numpy(), "lfilter_ss_states y", dtype=dtype)
        D.check(zf2.cpu().numpy(), zf1.cpu().numpy(), "lfilter_ss_states zf", dtype=dtype)
        res_hs = torch.ops.philtorch.lfilter_ss_backward(_t(b), _t(a), _t(zi), _t(x), _t(gy), _t(gzf), form, rev, hs)
        for r0, r1 in zip(res, res_hs):
            assert torch.equal(r0, r1)
        tb, ta, tz, tx = (_t(v.astype(np.float64), "cpu", True) for v in (b, a, zi, x))
        xs = tx.flip(-1) if rev else tx
        y, zf = _ssm_lfilter(tb, ta, xs, tz, form=("tdf2", "df2")[form], unroll_factor=1)
        if rev:
            y = y.flip(-1)
        loss = (y * _t(gy.astype(np.float64), "cpu")).sum() + (zf * _t(gzf.astype(np.float64), "cpu")).sum()
        ref = [r.numpy() for r in torch.autograd.grad(loss, (tb, ta, tz, tx))]
        for nm, gg, rr in zip(("grad_b", "grad_a", "grad_zi", "grad_x"), got, ref):
            D.check(gg, rr, f"{nm} rev={rev}", dtype=dtype)


def test_api_takes_fused_route_with_coefficient_gradients(hip, monkeypatch):
    """lti.state_space and lti.lfilter (orders 1, 3, 4 and df2 biquads) keep
    the fused ops when coefficients need gradients; the backward runs the
    fused coefficient-gradient op, and gradcheck (first order: the fused
    op) and gradgradcheck (second order: the composite) pass."""
    import torch

    from philtorch_amd import lti
    from philtorch_amd.lti import filtering, ssm

    taken = []
    orig_gate = ssm._fused_ss_applies
    monkeypatch.setattr(ssm, "_fused_ss_applies", lambda *a: taken.append(orig_gate(*a)) or taken[-1])
    orig_lgate = filtering._fused_lfilter_applies
    monkeypatch.setattr(filtering, "_fused_lfilter_applies", lambda *a: taken.append(orig_lgate(*a)) or taken[-1])

    g = D.rng(D.seed_of("api-ss-grad"))
    Bn, T, M = 2, 3001, 3
    A, b, c, d = (_t(v, rg=True) for v in _stable_model(g, M, ()))
    x = _t(g.standard_normal((Bn, T)), rg=True)
    y = lti.state_space(A, x, B=b, C=c, D=d, unroll_factor=1)
    assert taken[-1] is True
    gy = torch.randn_like(y)
    grads = torch.autograd.grad(y, (A, b, c, d, x), gy)
    ref = _composite_grads([A.detach().cpu().numpy(), b.detach().cpu().numpy(), c.detach().cpu().numpy(),
                            d.detach().cpu().numpy(), np.zeros((Bn, M)), x.detach().cpu().numpy()],
                           gy.cpu().numpy(), np.zeros((Bn, M)), 0, False, "cpu")
    for gg, rr, nm in zip(grads, [ref[0], ref[1], ref[2], ref[3], ref[5]], "AbcDx"):
        D.check(gg.cpu().numpy(), rr, f"state_space grad {nm}")
    for nb, na, form in ((2, 1, "tdf2"), (4, 3, "tdf2"), (5, 4, "df2"), (3, 2, "df2")):
        bb = _t(g.standard_normal((Bn, nb)), rg=True)
        aa = _t(np.ascontiguousarray(_lfilter_operands(g, nb, na, Bn, 2, False, np.float64)[1]), rg=True)
        yy = lti.lfilter(bb, aa, x, form=form, unroll_factor=1)
        assert taken[-1] is True, (nb, na, form)
        gb, ga = torch.autograd.grad(yy.sum(), (bb, aa))
        assert torch.isfinite(gb).all() and torch.isfinite(ga).all()
    # gradcheck (first order: the fused op) and gradgradcheck (the composite)
    As, bs, cs, ds = (_t(v, rg=True) for v in _stable_model(g, 2, (2,)))
    xs = _t(g.standard_normal((2, 40)), rg=True)
    f = lambda A_, b_, c_, d_, x_: torch.ops.philtorch.lti_ss(A_, b_, c_, d_, None, x_, 0)[0]  # noqa: E731
    assert torch.autograd.gradcheck(f, (As, bs, cs, ds, xs))
    assert torch.autograd.gradgradcheck(f, (As, bs, cs, ds, xs))
    bf = _t(g.standard_normal((2, 4)), rg=True)
    af = _t(np.ascontiguousarray(_lfilter_operands(g, 4, 3, 2, 2, False, np.float64)[1]), rg=True)
    for form in (0, 1):
        for rev in (False, True):
            fl = lambda b_, a_, x_: torch.ops.philtorch.lfilter_ss(b_, a_, None, x_, form, rev)[0]  # noqa: E731
            assert torch.autograd.gradcheck(fl, (bf, af, xs))
            # the states-keeping forwards the API takes with coefficient gradients
            fs = lambda b_, a_, x_: torch.ops.philtorch.lfilter_ss_states(b_, a_, None, x_, form, rev)[0]  # noqa: E731
            assert torch.autograd.gradcheck(fs, (bf, af, xs))
    fs = lambda A_, b_, c_, d_, x_: torch.ops.philtorch.lti_ss_states(A_, b_, c_, d_, None, x_, 0)[0]  # noqa: E731
    assert torch.autograd.gradcheck(fs, (As, bs, cs, ds, xs))
    det = [t.detach() for t in (bf, af)]
    torch.library.opcheck(torch.ops.philtorch.lfilter_ss_states.default, (*det, None, xs.detach(), 0, False))
    torch.library.opcheck(torch.ops.philtorch.lti_ss_states.default,
                          (As.detach(), bs.detach(), cs.detach(), ds.detach(), None, xs.detach(), 0, False))


def test_backward_ops_on_empty_inputs(hip):
    """The fused coefficient-gradient ops on rows of no steps (T = 0: zero
    coefficient gradients, grad_zi = grad_zf) and on no rows (B = 0)."""
    import torch

    g = D.rng(D.seed_of("grad-empty"))
    for B in (3, 0):
        M = 2
        A = _t(np.asarray(_normal_model(g, M, ()), np.float32))
        b, c = _t(g.standard_normal(M).astype(np.float32)), _t(g.standard_normal((B, M)).astype(np.float32))
        d = _t(g.standard_normal(B).astype(np.float32))
        zi, gzf = _t(g.standard_normal((B, M)).astype(np.float32)), _t(g.standard_normal((B, M)).astype(np.float32))
        x = torch.zeros(B, 0, device="cuda")
        gA, gb, gc, gd, gzi, gx = torch.ops.philtorch.lti_ss_backward(A, b, c, d, zi, x, x, gzf, 0, False)
        assert gx.shape == (B, 0) and gzi.shape == (B, M)
        assert torch.equal(gzi, gzf)
        for t in (gA, gb, gc, gd):
            assert t.numel() == 0 or torch.count_nonzero(t).item() == 0
        fb = _t(g.standard_normal((B, 3)).astype(np.float32))
        fa = _t(np.tile(np.asarray([-0.5, 0.2], np.float32), (B, 1)))
        gb2, ga2, gzi2, gx2 = torch.ops.philtorch.lfilter_ss_backward(fb, fa, zi, x, x, gzf, 0, False)
        assert torch.equal(gzi2, gzf) and gx2.shape == (B, 0)
        assert torch.count_nonzero(gb2).item() == 0 and torch.count_nonzero(ga2).item() == 0
        Al = torch.zeros(B, 0, M, M, device="cuda")
        bl = _t(g.standard_normal((B, 1, M)).astype(np.float32))
        res = torch.ops.philtorch.lpv_ss_backward(Al, bl, None, None, zi, x, x, gzf, 0, False, False)
        assert torch.equal(res[4], gzf) and res[0].shape == (B, 0, M, M)
        assert torch.count_nonzero(res[1]).item() == 0
