"""GPU parity of the fused single-input, single-output LPV state space
(phs_lpv_ss_fwd, op philtorch::lpv_ss, the route of philtorch_amd.lpv.
state_space for such models of order <= 4 when no gradient is wanted).

The C ABI entry point (ctypes, raw device pointers, the caller's stream)
against oracle.lpv_state_space (B x, the LPV scan, the state shift,
C h + D x; pinned to the per-step loop and to the LTI model in
tests/test_oracle.py), evaluated in fp64 on the GPU's exact inputs: orders 1
to 4, fp32 and fp64, every layout of b, c and d (shared, per row, per step,
per row and step, absent / out_idx), shared and per-row A, rows shorter than
a lane's chunk, on and around tile edges and of a million steps, the forced
look-back fallback.  Through the torch API: the reference's shape cases
(including the ambiguous ones, which follow its match order), gradients
(the composite route) and opcheck.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import _data as D

pytestmark = pytest.mark.gpu

FLOATS = [np.float32, np.float64]
SHAPES = [(1, 1), (2, 7), (3, 383), (2, 1536), (3, 1537), (2, 3072), (2, 3073), (2, 20001)]


@pytest.fixture(scope="module")
def api(hip):
    import torch

    from tests import capi

    lib = capi.load()
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    yield lib, ws, capi
    lib.phs_debug_set_spin_limit(0)


def _dev(v):
    import torch

    return None if v is None else torch.from_numpy(np.ascontiguousarray(v)).cuda()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _strides(v, T, width):
    """(row, step) element strides of a (1 | B, 1 | T, width...) operand."""
    if v is None:
        return 0, 0
    rows, steps = v.shape[0], v.shape[1]
    return (0 if rows == 1 else steps * width), (0 if steps == 1 else width)


def _run(api, A, b, c, d, zi, x, out_idx=0, rev=False, transposed=False):
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    Bn, T = x.shape
    M = A.shape[-1]
    need = lib.phs_lpv_ss_workspace_size(dt, M, Bn, T)
    assert 0 < need <= ws.numel()
    tA, tb, tc, td, tz, tx = (_dev(v) for v in (A, b, c, d, zi, x))
    y = torch.full_like(tx, float("nan"))
    zf = torch.full((Bn, M), float("nan"), dtype=tx.dtype, device="cuda")
    flags = (capi.PHS_LPV_A_SHARED if A.ndim == 3 else 0) | (capi.PHS_LPV_A_TRANSPOSED if transposed else 0)
    print(f"lpv_ss capi M={M} B={Bn} T={T} rev={rev} A_flags={flags}", flush=True)
    rc = (lib.phs_lpv_ss_rev if rev else lib.phs_lpv_ss_fwd)(dt, M, Bn, T, _p(tA), flags, _p(tb), *_strides(b, T, M), _p(tc),
                            *_strides(c, T, M), out_idx, _p(td), *_strides(d, T, 1), _p(tz), _p(tx), _p(y), _p(zf),
                            _p(ws), need, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    return y.cpu().numpy(), zf.cpu().numpy()


def _model(g, M, Bn, T, A_shared):
    """Stable time-varying A: per step a block diagonal of scaled 2x2
    rotations (and a real pole for odd M), radius < 0.98, turned dense by a
    fixed orthogonal basis for M > 2 (orthogonal similarity keeps every
    step's norm below 1)."""
    lead = (T,) if A_shared else (Bn, T)
    if M == 1:
        return g.uniform(-0.98, 0.98, lead + (1, 1))
    A = np.zeros(lead + (M, M))
    for i in range(0, M - 1, 2):
        r = g.uniform(0.5, 0.98, lead)
        th = g.uniform(0, np.pi, lead)
        A[..., i, i] = r * np.cos(th)
        A[..., i, i + 1] = -r * np.sin(th)
        A[..., i + 1, i] = r * np.sin(th)
        A[..., i + 1, i + 1] = r * np.cos(th)
    if M % 2:
        A[..., M - 1, M - 1] = g.uniform(-0.98, 0.98, lead)
    if M > 2:
        Q, _ = np.linalg.qr(g.standard_normal((M, M)))
        A = Q @ A @ Q.T
    return A


def _layout(g, kind, Bn, T, width):
    shape = {"shared": (1, 1), "row": (Bn, 1), "step": (1, T), "rowstep": (Bn, T)}[kind]
    return g.standard_normal(shape + ((width,) if width else ()))


def _check(got, A, b, c, d, zi, x, out_idx, dtype, name, rev=False):
    """Against the oracle; rev: the model over the time-flipped row and
    operands, flipped back."""
    w = lambda v: None if v is None else np.asarray(v, np.float64)  # noqa: E731
    if rev:
        ft = lambda v, ax: v if v is None or v.shape[ax] == 1 else np.ascontiguousarray(np.flip(v, ax))  # noqa: E731
        A, b, c, d, x = ft(A, -3), ft(b, 1), ft(c, 1), ft(d, 1), np.ascontiguousarray(np.flip(x, 1))
    ry, rzf = oracle.lpv_state_space(w(A), w(x), w(b), w(c), w(d), w(zi), out_idx=out_idx)
    if rev:
        ry = np.ascontiguousarray(ry[:, ::-1])
    D.check(got[0], ry, f"{name} y", dtype=dtype)
    D.check(got[1], rzf, f"{name} zf", dtype=dtype, scale=np.max(np.abs(ry)) if ry.size else None)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("Bn,T", SHAPES)
def test_lpv_ss_capi_parity(api, dtype, M, Bn, T):
    g = D.rng(D.seed_of("lpv-ss", dtype, M, Bn, T))
    x = g.standard_normal((Bn, T)).astype(dtype)
    zi = g.standard_normal((Bn, M)).astype(dtype)
    cast = lambda v: None if v is None else v.astype(dtype)  # noqa: E731
    for A_shared, kb, kc, kd in ((False, "rowstep", "rowstep", "rowstep"), (True, "shared", "step", "row"),
                                 (False, "step", "row", "shared"), (True, "row", "shared", "step"),
                                 (False, None, None, None)):
        A = cast(_model(g, M, Bn, T, A_shared))
        b = cast(_layout(g, kb, Bn, T, M)) if kb else None
        c = cast(_layout(g, kc, Bn, T, M)) if kc else None
        d = cast(_layout(g, kd, Bn, T, 0)) if kd else None
        idx = M - 1
        name = f"M={M} B={Bn} T={T} A_shared={A_shared} b={kb} c={kc} d={kd}"
        _check(_run(api, A, b, c, d, zi, x, out_idx=idx), A, b, c, d, zi, x, idx, dtype, name)
        _check(_run(api, A, b, c, d, zi, x, out_idx=idx, rev=True), A, b, c, d, zi, x, idx, dtype, name + " rev",
               rev=True)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_lpv_ss_capi_long_rows_and_fallback(api, dtype, M):
    lib = api[0]
    g = D.rng(D.seed_of("lpv-ss-long", dtype, M))
    Bn, T = 2, 1_000_003
    A = _model(g, M, Bn, T, False).astype(dtype)
    b, c, d = (_layout(g, "rowstep", Bn, T, w).astype(dtype) for w in (M, M, 0))
    x = g.standard_normal((Bn, T)).astype(dtype)
    zi = g.standard_normal((Bn, M)).astype(dtype)
    _check(_run(api, A, b, c, d, zi, x), A, b, c, d, zi, x, 0, dtype, "long rows")
    xs = x[:, :40000].copy()
    As, bs, cs, ds = A[:, :40000].copy(), b[:, :40000].copy(), c[:, :40000].copy(), d[:, :40000].copy()
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, As, bs, cs, ds, zi, xs)
        got_rev = _run(api, As, bs, cs, ds, zi, xs, rev=True)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(got, As, bs, cs, ds, zi, xs, 0, dtype, "fallback")
    _check(got_rev, As, bs, cs, ds, zi, xs, 0, dtype, "rev fallback", rev=True)


def test_lpv_ss_capi_errors(api):
    lib, ws, capi = api
    d = ctypes.c_void_p(16)

    def call(M=2, B=2, T=100, c=d, out_idx=0, rs=0, wsb=1 << 30, dt=0):
        return lib.phs_lpv_ss_fwd(dt, M, B, T, d, 1, None, rs, 0, c, 0, 0, out_idx, None, 0, 0, None, d, d, None, d,
                                  wsb, None)

    assert call(dt=2) == capi.PHS_ERR_DTYPE
    assert call(M=5) == capi.PHS_ERR_INVALID
    assert call(c=None, out_idx=2) == capi.PHS_ERR_INVALID
    assert call(rs=-1) == capi.PHS_ERR_INVALID
    assert call(wsb=lib.phs_lpv_ss_workspace_size(0, 2, 2, 100) - 1) == capi.PHS_ERR_WORKSPACE
    assert call(B=0) == capi.PHS_OK and call(T=0) == capi.PHS_OK


def test_lpv_state_space_api_routes_and_shapes(hip, monkeypatch):
    """lpv.state_space on HIP with unroll_factor=1 takes philtorch::lpv_ss for
    the reference's single-output shape cases and matches the composed
    route (the same call with the fused route switched off); multi-output
    shapes keep the composed route."""
    import torch

    from philtorch_amd.lpv import ssm

    g = D.rng(D.seed_of("lpv-ss-api"))
    Bn, T, M = 3, 3000, 2
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda")  # noqa: E731
    A = t(_model(g, M, Bn, T, False))
    x = t(g.standard_normal((Bn, T)))
    zi = t(g.standard_normal((Bn, M)))
    cases = [dict(B=t(g.standard_normal(M)), C=t(g.standard_normal(M)), D=t(g.standard_normal(()))),
             dict(B=t(g.standard_normal((T, M))), C=t(g.standard_normal((Bn, M))), D=t(g.standard_normal(T))),
             dict(B=t(g.standard_normal((Bn, T, M))), C=t(g.standard_normal((Bn, T, M))),
                  D=t(g.standard_normal((Bn, T)))),
             dict(B=None, C=None, D=t(g.standard_normal(Bn)), out_idx=1),
             dict(B=t(g.standard_normal((Bn, M))), C=t(g.standard_normal((T, M))), D=None)]
    taken = []
    orig = ssm._fused_lpv_ss_applies
    monkeypatch.setattr(ssm, "_fused_lpv_ss_applies", lambda *a: taken.append(orig(*a)) or taken[-1])
    for i, kw in enumerate(cases):
        for z in (zi, None):
            out = hip.lpv.state_space(A, x, zi=z, unroll_factor=1, **kw)
            assert taken[-1] is True, i
            monkeypatch.setattr(ssm, "_fused_lpv_ss_applies", lambda *a: False)
            ref = hip.lpv.state_space(A, x, zi=z, unroll_factor=1, **kw)
            monkeypatch.setattr(ssm, "_fused_lpv_ss_applies", lambda *a: taken.append(orig(*a)) or taken[-1])
            if z is None:
                out, ref = (out,), (ref,)
            for o, r in zip(out, ref):
                D.check(o.cpu().numpy(), r.cpu().numpy(), f"case {i} zi={z is not None}")
    # multi-output C (one row per output) and a state output keep the composed route
    hip.lpv.state_space(A, x, C=t(g.standard_normal((4, M))), unroll_factor=1)
    assert taken[-1] is False
    hip.lpv.state_space(A, x, unroll_factor=1)
    assert taken[-1] is False


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_lpv_state_space_signal_gradient_takes_adjoint_pass(hip, monkeypatch, dtype, M):
    """lpv.state_space with only x and zi requiring grad runs the fused
    route forward and its adjoint (A[t]^T read in place, c and b swapped,
    reversed in time) backward; gradients against the composed route's
    autograd."""
    import torch

    from philtorch_amd.lpv import ssm

    g = D.rng(D.seed_of("lpv-ss-adjoint", dtype, M))
    Bn, T = 3, 5000
    t = lambda v: torch.tensor(np.asarray(v, dtype), device="cuda")  # noqa: E731
    A = t(_model(g, M, Bn, T, False))
    b, c, d = t(g.standard_normal((Bn, T, M))), t(g.standard_normal(M)), t(g.standard_normal((Bn, T)))
    x0, z0 = g.standard_normal((Bn, T)), g.standard_normal((Bn, M))
    gy, gzf = t(g.standard_normal((Bn, T))), t(g.standard_normal((Bn, M)))
    taken = []
    orig = ssm._fused_lpv_ss_applies
    res = []
    for fused in (True, False):
        monkeypatch.setattr(ssm, "_fused_lpv_ss_applies",
                            (lambda *a: taken.append(orig(*a)) or taken[-1]) if fused else (lambda *a: False))
        for kw in (dict(C=c), dict(out_idx=M - 1)):
            x, z = t(x0).requires_grad_(True), t(z0).requires_grad_(True)
            y, zf = hip.lpv.state_space(A, x, B=b, D=d, zi=z, unroll_factor=1, **kw)
            ((y * gy).sum() + (zf * gzf).sum()).backward()
            res.append((x.grad.cpu().numpy(), z.grad.cpu().numpy()))
    assert taken == [True, True]
    for i in range(2):
        D.check(res[i][0], res[i + 2][0], f"grad_x {i}", dtype=dtype)
        D.check(res[i][1], res[i + 2][1], f"grad_zi {i}", dtype=dtype, scale=np.max(np.abs(res[i + 2][0])))


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("rev", [False, True])
def test_lpv_ss_capi_transposed_A(api, dtype, M, rev):
    """PHS_LPV_A_TRANSPOSED reads each step's matrix transposed where it
    lies: bit for bit the result of passing the transposed copy, per-row and
    shared A, through the look-back (T spans many tiles), and against the
    oracle on the transposed model."""
    g = D.rng(D.seed_of("lpv-ss-transposed", dtype, M, rev))
    Bn, T = 3, 40_001
    x = g.standard_normal((Bn, T)).astype(dtype)
    zi = g.standard_normal((Bn, M)).astype(dtype)
    b, c, d = _layout(g, "rowstep", Bn, T, M), _layout(g, "row", Bn, T, M), _layout(g, "step", Bn, T, 0)
    b, c, d = (v.astype(dtype) for v in (b, c, d))
    for shared in (False, True):
        A = _model(g, M, Bn, T, shared).astype(dtype)  # rotations: A^T != A for M > 1
        At = np.ascontiguousarray(np.swapaxes(A, -1, -2))
        got = _run(api, A, b, c, d, zi, x, rev=rev, transposed=True)
        ref = _run(api, At, b, c, d, zi, x, rev=rev)
        np.testing.assert_array_equal(got[0], ref[0])
        np.testing.assert_array_equal(got[1], ref[1])
        _check(got, At, b, c, d, zi, x, 0, dtype, f"transposed shared={shared}", rev=rev)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_lpv_ss_reversed_op_gradients(hip, M):
    import torch

    g = D.rng(D.seed_of("lpv-ss-rev-grad", M))
    Bn, T = 2, 20
    t = lambda v, rg=False: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=rg)  # noqa: E731
    A = t(_model(g, M, Bn, T, False))
    b, c, d = t(g.standard_normal((Bn, T, M))), t(g.standard_normal((1, 1, M))), t(g.standard_normal((Bn, 1)))
    x, zi = t(g.standard_normal((Bn, T)), True), t(g.standard_normal((Bn, M)), True)
    for rev in (False, True):
        f = lambda z_, x_: torch.ops.philtorch.lpv_ss(A, b, c, d, z_, x_, 0, rev)  # noqa: E731
        assert torch.autograd.gradcheck(f, (zi, x))
        assert torch.autograd.gradgradcheck(f, (zi, x))
        f2 = lambda z_, x_: torch.ops.philtorch.lpv_ss(A, None, None, d, z_, x_, M - 1, rev)  # noqa: E731
        assert torch.autograd.gradcheck(f2, (zi, x))
        # the transposed model: the adjoint pass then reads A as it lies
        f3 = lambda z_, x_: torch.ops.philtorch.lpv_ss(A, b, c, d, z_, x_, 0, rev, True)  # noqa: E731
        assert torch.autograd.gradcheck(f3, (zi, x))
        assert torch.autograd.gradgradcheck(f3, (zi, x))
    Ag, bg = A.clone().requires_grad_(True), b.clone().requires_grad_(True)
    fA = lambda A_, b_, x_: torch.ops.philtorch.lpv_ss(A_, b_, c, d, None, x_, 0, True)[0]  # noqa: E731
    assert torch.autograd.gradcheck(fA, (Ag, bg, x))
    fAt = lambda A_, b_, x_: torch.ops.philtorch.lpv_ss(A_, b_, c, d, None, x_, 0, False, True)[0]  # noqa: E731
    assert torch.autograd.gradcheck(fAt, (Ag, bg, x))
    yt, zft = torch.ops.philtorch.lpv_ss(A, b, c, d, zi, x, 0, False, True)
    yc, zfc = torch.ops.philtorch.lpv_ss(A.mT.contiguous(), b, c, d, zi, x, 0)
    assert torch.equal(yt, yc) and torch.equal(zft, zfc)
    y, zf = torch.ops.philtorch.lpv_ss(A, b, c, d, zi, x, 0, True)
    yr, zfr = torch.ops.philtorch.lpv_ss(A.flip(-3), b.flip(1), c, d, zi, x.flip(-1), 0)
    D.check(y.detach().cpu().numpy(), yr.flip(-1).detach().cpu().numpy(), "reverse y")
    D.check(zf.detach().cpu().numpy(), zfr.detach().cpu().numpy(), "reverse zf")


def test_lpv_ss_op_gradients_and_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("lpv-ss-grad"))
    Bn, T, M = 2, 20, 2
    t = lambda v, rg=False: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=rg)  # noqa: E731
    A = t(_model(g, M, Bn, T, False), True)
    b, c = t(g.standard_normal((Bn, T, M)), True), t(g.standard_normal((1, 1, M)), True)
    d = t(g.standard_normal((Bn, 1)), True)
    x, zi = t(g.standard_normal((Bn, T)), True), t(g.standard_normal((Bn, M)), True)
    f = lambda *a: torch.ops.philtorch.lpv_ss(*a, 0)  # noqa: E731
    assert torch.autograd.gradcheck(f, (A, b, c, d, zi, x))
    f2 = lambda A_, x_, z_: torch.ops.philtorch.lpv_ss(A_, None, None, None, z_, x_, 1)  # noqa: E731
    assert torch.autograd.gradcheck(f2, (A, x, zi))
    s = lambda v: torch.tensor(np.asarray(v, np.float32), device="cuda")  # noqa: E731
    torch.library.opcheck(torch.ops.philtorch.lpv_ss.default,
                          (s(_model(g, M, Bn, 500, True)), s(g.standard_normal((1, 500, M))), None,
                           s(g.standard_normal((1, 1))), None, s(g.standard_normal((Bn, 500))), 1),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    torch.library.opcheck(torch.ops.philtorch.lpv_ss.default,
                          (s(_model(g, M, Bn, 500, False)), None, s(g.standard_normal((Bn, 1, M))), None,
                           s(g.standard_normal((Bn, M))), s(g.standard_normal((Bn, 500))), 0, True),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 2, 4])
def test_lpv_ss_capi_aggregates_only_multi_window(api, dtype, M):
    """Tiles after a row's first publish aggregates only (testing hook): every
    look-back folds back to tile 0 through several 64-tile windows."""
    lib = api[0]
    g = D.rng(D.seed_of("lpv-ss-agg-only", dtype, M))
    Bn, T = 2, 300_007
    A = _model(g, M, Bn, T, False).astype(dtype)
    b, c, d = (_layout(g, "rowstep", Bn, T, w).astype(dtype) for w in (M, M, 0))
    x = g.standard_normal((Bn, T)).astype(dtype)
    zi = g.standard_normal((Bn, M)).astype(dtype)
    lib.phs_debug_set_aggregates_only(1)
    try:
        got = _run(api, A, b, c, d, zi, x)
        got_rev = _run(api, A, b, c, d, zi, x, rev=True)
    finally:
        lib.phs_debug_set_aggregates_only(0)
    _check(got, A, b, c, d, zi, x, 0, dtype, "aggregates only")
    _check(got_rev, A, b, c, d, zi, x, 0, dtype, "aggregates only rev", rev=True)
