"""GPU parity of the fused coefficient gradients of the single-input
single-output LPV state space (phs_lpv_ss_bwd, philtorch::lpv_ss_backward).

Pins:

* directional derivatives of the oracle (oracle.lpv_state_space, pinned to
  the per-step loop and to the LTI model in tests/test_oracle.py): for a
  random direction V of each input, grad . V against the central difference
  of L = <g, y> + <g_zf, zf> evaluated by the oracle in fp64 (L is linear in
  each of b, c, d, zi and x, so those differences are exact for any step and
  take a large one; A's a small one);
* the autograd of the composed route the fused kernels replace (B x, the
  native LPV scan, the state shift, C h + D x; philtorch/lpv/ssm.py:337-581)
  on the same inputs, fp32 and fp64, orders 1-4, every layout of b, c and d
  (shared, per row, per step, per row and step, absent / out_idx), shared
  and per-row A, A read transposed, forward and reversed calls, rows of one
  step, on and around a tile and of many tiles;
* the API: lpv.state_space keeps the fused route when coefficients need
  gradients (its forward then keeps its states, philtorch::lpv_ss_states,
  whose outputs and backward are checked bit-exact against lpv_ss's);
  gradcheck (the fused ops) and gradgradcheck (the composite).
"""
import numpy as np
import pytest

import oracle
from tests import _data as D
from tests.test_gpu_lpv_ss import _layout, _model

pytestmark = pytest.mark.gpu

FLOATS = [np.float32, np.float64]
ORDERS = [1, 2, 3, 4]
# (A shared, b, c, d)
LAYOUTS = [(False, "rowstep", "rowstep", "rowstep"), (True, "shared", "step", "row"), (False, "step", "row", "shared"),
           (True, "row", "shared", "step"), (False, None, None, None), (True, "rowstep", None, "rowstep"),
           (False, None, "rowstep", None)]


def _operands(g, M, Bn, T, layout, dtype):
    A_sh, kb, kc, kd = layout
    A = _model(g, M, Bn, T, A_sh)
    b = None if kb is None else _layout(g, kb, Bn, T, M)
    c = None if kc is None else _layout(g, kc, Bn, T, M)
    d = None if kd is None else _layout(g, kd, Bn, T, 0)
    zi = g.standard_normal((Bn, M))
    x = g.standard_normal((Bn, T))
    cast = lambda v: None if v is None else np.ascontiguousarray(v, dtype=dtype)  # noqa: E731
    return [cast(v) for v in (A, b, c, d, zi, x)]


def _t(v, dev="cuda", rg=False):
    import torch

    return None if v is None else torch.tensor(v, device=dev, requires_grad=rg)


def _oracle_loss(ops, gy, gzf, out_idx, rev):
    A, b, c, d, zi, x = ops
    if rev:
        ft = lambda v, ax: v if v is None or v.shape[ax] == 1 else np.ascontiguousarray(np.flip(v, ax))  # noqa: E731
        A, b, c, d, x = ft(A, -3), ft(b, 1), ft(c, 1), ft(d, 1), np.ascontiguousarray(x[:, ::-1])
    y, zf = oracle.lpv_state_space(A, x, b, c, d, zi, out_idx=out_idx)
    if rev:
        y = y[:, ::-1]
    return float(np.sum(gy * y) + np.sum(gzf * zf))


@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: "-".join(str(v) for v in l))
@pytest.mark.parametrize("rev", [False, True])
def test_lpv_ss_backward_directional_derivative_vs_oracle(hip, M, layout, rev):
    import torch

    g = D.rng(D.seed_of("lpv-grad-fd", M, layout, rev))
    Bn, T = 3, 4001  # several tiles per row (384-3072 steps by order)
    ops = _operands(g, M, Bn, T, layout, np.float64)
    out_idx = M - 1
    gy, gzf = g.standard_normal((Bn, T)), g.standard_normal((Bn, M))
    print(f"lpv_ss_backward fd M={M} layout={layout} rev={rev}", flush=True)
    res = torch.ops.philtorch.lpv_ss_backward(*[_t(v) for v in ops], _t(gy), _t(gzf), out_idx, rev)
    grads = [r.cpu().numpy() for r in res]
    for i in range(6):
        if ops[i] is None:
            assert grads[i].size == 0
            continue
        assert grads[i].shape == ops[i].shape
        V = g.standard_normal(ops[i].shape)
        eps, rtol = (1e-6, 1e-5) if i == 0 else (1.0, 1e-7)
        p = [v if j != i else v + eps * V for j, v in enumerate(ops)]
        m = [v if j != i else v - eps * V for j, v in enumerate(ops)]
        fdi = (_oracle_loss(p, gy, gzf, out_idx, rev) - _oracle_loss(m, gy, gzf, out_idx, rev)) / (2 * eps)
        pi = float(np.sum(grads[i] * V))
        assert abs(pi - fdi) <= rtol * max(1.0, abs(fdi)), (i, pi, fdi)


def _composite_grads(ops, gy, gzf, out_idx, rev, transpose_A=False):
    """Autograd of the composed route on the CPU in fp64."""
    import torch

    from philtorch_amd.lpv.ssm import _lpv_state_space_composite

    ts = [_t(v, "cpu", v is not None) for v in ops]
    A, b, c, d, zi, x = ts
    Am = A.mT if transpose_A else A
    if rev:
        ft = lambda v, ax: v if v is None or v.size(ax) == 1 else v.flip(ax)  # noqa: E731
        y, zf = _lpv_state_space_composite(Am.flip(-3), ft(b, 1), ft(c, 1), ft(d, 1), zi, x.flip(-1),
                                           out_idx=out_idx)
        y = y.flip(-1)
    else:
        y, zf = _lpv_state_space_composite(Am, b, c, d, zi, x, out_idx=out_idx)
    loss = (y * _t(gy, "cpu")).sum() + (zf * _t(gzf, "cpu")).sum()
    wrt = [t for t in ts if t is not None]
    gr = torch.autograd.grad(loss, wrt)
    out, k = [], 0
    for t in ts:
        out.append(None if t is None else gr[k].numpy())
        k += t is not None
    return out


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("Bn,T", [(2, 1), (3, 383), (2, 1536), (3, 1537), (2, 3072), (2, 20001)])
def test_lpv_ss_backward_vs_composed_route(hip, dtype, M, Bn, T):
    import torch

    for li, layout in enumerate(LAYOUTS):
        for rev, tr in ((False, False), (True, False), (False, True)):
            g = D.rng(D.seed_of("lpv-grad-comp", np.dtype(dtype).str, M, Bn, T, li, rev, tr))
            ops = _operands(g, M, Bn, T, layout, dtype)
            out_idx = 0 if M == 1 else 1
            gy = g.standard_normal((Bn, T)).astype(dtype)
            gzf = g.standard_normal((Bn, M)).astype(dtype)
            print(f"lpv_ss_backward {np.dtype(dtype).name} M={M} B={Bn} T={T} layout={layout} rev={rev} "
                  f"transpose_A={tr}", flush=True)
            res = torch.ops.philtorch.lpv_ss_backward(*[_t(v) for v in ops], _t(gy), _t(gzf), out_idx, rev, tr)
            got = [r.cpu().numpy() for r in res]
            # the forward keeping its states (phs_lpv_ss_fwd_hs) gives lpv_ss's outputs, and the
            # backward given them (phs_lpv_ss_bwd_hs) the same gradients, bit for bit
            y1, zf1 = torch.ops.philtorch.lpv_ss(*[_t(v) for v in ops], out_idx, rev, tr)
            y2, zf2, hs = torch.ops.philtorch.lpv_ss_states(*[_t(v) for v in ops], out_idx, rev, tr)
            assert hs.shape == (Bn, T, M) and torch.equal(y1, y2) and torch.equal(zf1, zf2)
            res_hs = torch.ops.philtorch.lpv_ss_backward(*[_t(v) for v in ops], _t(gy), _t(gzf), out_idx, rev, tr,
                                                         hs)
            for r0, r1 in zip(res, res_hs):
                assert torch.equal(r0, r1)
            ref = _composite_grads([None if v is None else v.astype(np.float64) for v in ops],
                                   gy.astype(np.float64), gzf.astype(np.float64), out_idx, rev, tr)
            for i, nm in enumerate(("grad_A", "grad_B", "grad_C", "grad_D", "grad_zi", "grad_x")):
                if ops[i] is None:
                    assert got[i].size == 0
                    continue
                D.check(got[i], ref[i], f"{nm} layout={layout} rev={rev} transpose_A={tr}", dtype=dtype)


def test_lpv_api_takes_fused_route_with_coefficient_gradients(hip, monkeypatch):
    import torch

    from philtorch_amd import lpv
    from philtorch_amd.lpv import ssm

    taken = []
    orig = ssm._fused_lpv_ss_applies
    monkeypatch.setattr(ssm, "_fused_lpv_ss_applies", lambda *a: taken.append(orig(*a)) or taken[-1])
    g = D.rng(D.seed_of("lpv-api-grad"))
    Bn, T, M = 3, 5000, 2
    A = _t(_model(g, M, Bn, T, False), rg=True)
    b = _t(g.standard_normal((Bn, T, M)), rg=True)
    c = _t(g.standard_normal(M), rg=True)
    d = _t(g.standard_normal((Bn, T)), rg=True)
    x = _t(g.standard_normal((Bn, T)), rg=True)
    zi = _t(g.standard_normal((Bn, M)), rg=True)
    y, zf = lpv.state_space(A, x, B=b, C=c, D=d, zi=zi, unroll_factor=1)
    assert taken[-1] is True
    gy, gzf = torch.randn_like(y), torch.randn_like(zf)
    grads = torch.autograd.grad((y, zf), (A, b, c, d, zi, x), (gy, gzf))
    ref = _composite_grads([t.detach().cpu().numpy() for t in (A, b, c.reshape(1, 1, M), d, zi, x)],
                           gy.cpu().numpy(), gzf.cpu().numpy(), None, False)
    ref[2] = ref[2].reshape(M)
    for gg, rr, nm in zip(grads, ref, ("A", "B", "C", "D", "zi", "x")):
        D.check(gg.cpu().numpy(), rr, f"state_space grad {nm}")
    # gradcheck through the fused op (first order), gradgradcheck through the composite
    Bs, Ts = 2, 30
    As = _t(_model(g, M, Bs, Ts, True), rg=True)
    bs, cs = _t(g.standard_normal((1, Ts, M)), rg=True), _t(g.standard_normal((Bs, 1, M)), rg=True)
    ds, xs = _t(g.standard_normal((1, 1)), rg=True), _t(g.standard_normal((Bs, Ts)), rg=True)
    zs = _t(g.standard_normal((Bs, M)), rg=True)
    for rev in (False, True):
        for tr in (False, True):
            f = lambda *a: torch.ops.philtorch.lpv_ss(*a, 0, rev, tr)  # noqa: E731
            assert torch.autograd.gradcheck(f, (As, bs, cs, ds, zs, xs))
    f = lambda *a: torch.ops.philtorch.lpv_ss(*a, 0)  # noqa: E731
    assert torch.autograd.gradgradcheck(f, (As, bs, cs, ds, zs, xs))
    # the states-keeping forward the API takes here: gradcheck of its (y, zf), and opcheck
    for rev in (False, True):
        f = lambda *a: torch.ops.philtorch.lpv_ss_states(*a, 0, rev)[:2]  # noqa: E731
        assert torch.autograd.gradcheck(f, (As, bs, cs, ds, zs, xs))
    det = [t.detach() for t in (As, bs, cs, ds, zs, xs)]
    torch.library.opcheck(torch.ops.philtorch.lpv_ss_states.default, (*det, 0, True, False))


def test_lpv_shared_step_gradients_above_scratch_limit_take_composite(hip, monkeypatch):
    """Operands shared by the rows and varying along time (A (T, M, M); b, d
    with one row): the fused backward would first write every row's
    per-step gradient.  Above lpv.ssm._LPV_ROW_SCRATCH_LIMIT bytes of that
    scratch the gradients come from the composed route's autograd instead;
    both routes' gradients agree (fp64), and the byte count is the fused
    backward's."""
    import torch

    from philtorch_amd import lpv
    from philtorch_amd.lpv import ssm

    g = D.rng(D.seed_of("lpv-scratch-limit"))
    Bn, T, M = 3, 7000, 3
    A0 = _model(g, M, Bn, T, True)
    b0, c0 = g.standard_normal((1, T, M)), g.standard_normal((Bn, 1, M))
    d0, x0, z0 = g.standard_normal((1, T)), g.standard_normal((Bn, T)), g.standard_normal((Bn, M))
    gy, gzf = g.standard_normal((Bn, T)), g.standard_normal((Bn, M))
    assert ssm._lpv_row_scratch_bytes(_t(A0), _t(b0), _t(c0), _t(d0), _t(x0), (True,) * 4) == Bn * T * (M * M + M + 1) * 8
    grads = {}
    for limit in (ssm._LPV_ROW_SCRATCH_LIMIT, 0):
        print(f"lpv scratch limit={limit}", flush=True)
        monkeypatch.setattr(ssm, "_LPV_ROW_SCRATCH_LIMIT", limit)
        # the API's shapes: B (T, M) and D (T,) shared by the rows, C (batch, M)
        ins = [_t(v, rg=True) for v in (A0, b0.reshape(T, M), c0.reshape(Bn, M), d0.reshape(T), z0, x0)]
        A, b, c, d, zi, x = ins
        y, zf = lpv.state_space(A, x, B=b, C=c, D=d, zi=zi, unroll_factor=1)
        grads[limit] = torch.autograd.grad((y, zf), ins, (_t(gy), _t(gzf)))
    for nm, a, r in zip(("A", "B", "C", "D", "zi", "x"), grads[0], grads[ssm._LPV_ROW_SCRATCH_LIMIT]):
        D.check(a.cpu().numpy(), r.cpu().numpy(), f"composite vs fused grad {nm}", dtype=np.float64)
