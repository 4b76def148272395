"""GPU parity of the fused single-input single-output LTI state space
(phs_lti_ss_fwd, op philtorch::lti_ss, the route of philtorch_amd.lti.
state_space and so of lti.lfilter for models of order <= 4).

The C ABI entry point (ctypes, raw device pointers, the caller's stream)
against oracle.lti_state_space (B x, the oracle's lti_recurN, the shifted
state sequence and C h + D x, as philtorch composes them; pinned to
scipy.signal.dlsim in tests/test_oracle.py), evaluated in fp64 on the GPU's
exact inputs.  Orders 1 to 4; dense stable A (a companion matrix in a random
basis); shared and per-row A, b, c, d; b absent (input into state 0), c
absent (out_idx), d absent; initial and final states; rows shorter than a
lane's chunk, on and around a tile (6144 fp32 steps, 3072 fp64; the
order-2 fp32 plain pass's 30720-step wide tile, both directions), of odd
length and of a million steps; the forced look-back fallback.  Through the
torch API: lfilter of orders 1, 3 and 4 in both forms against the CPU
(reference) route, state_space against its composed route, gradients
(first and second order, through the composite formula), the route choice
and opcheck.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import _data as D
from tests.test_oracle import _stable_model

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (2, 7), (3, 3071), (2, 3072), (2, 6143), (3, 6144), (2, 6145), (2, 20001)]
FLOATS = [np.float32, np.float64]
ORDERS = [1, 2, 3, 4]


@pytest.fixture(scope="module")
def api(hip):
    import torch

    from tests import capi

    lib = capi.load()
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    yield lib, ws, capi
    lib.phs_debug_set_spin_limit(0)


def _dev(x):
    import torch

    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _run(api, A, b, c, d, zi, x, out_idx=0, want_zf=True, rev=False):
    """phs_lti_ss_fwd (phs_lti_ss_rev) through the C ABI; numpy (y, zf)."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    Bn, T = x.shape
    M = A.shape[-1]
    need = lib.phs_lti_ss_workspace_size(dt, M, Bn, T)
    assert 0 < need <= ws.numel()
    tA, tb, tc, td, tz, tx = (_dev(v) for v in (A, b, c, d, zi, x))
    y = torch.full_like(tx, float("nan"))
    zf = torch.full((Bn, M), float("nan"), dtype=tx.dtype, device="cuda") if want_zf else None
    sh = lambda v, nd: int(v is not None and np.ndim(v) == nd)  # noqa: E731
    fn = lib.phs_lti_ss_rev if rev else lib.phs_lti_ss_fwd
    print(f"lti_ss capi M={M} B={Bn} T={T} rev={rev}", flush=True)
    rc = fn(dt, M, Bn, T, _p(tA), sh(A, 2), _p(tb), sh(b, 1), _p(tc), sh(c, 1), out_idx, _p(td),
            int(d is not None and np.size(d) == 1), _p(tz), _p(tx), _p(y), _p(zf), _p(ws), need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    return y.cpu().numpy(), None if zf is None else zf.cpu().numpy()


def _case(dtype, M, Bn, T, shared, seed):
    g = D.rng(seed)
    A, b, c, d = _stable_model(g, M, () if shared else (Bn,))
    x = g.standard_normal((Bn, T))
    zi = g.standard_normal((Bn, M))
    cast = lambda v: None if v is None else np.asarray(v).astype(dtype)  # noqa: E731
    return [cast(v) for v in (A, b, c, np.reshape(d, (1,)) if shared else d, zi, x)]


def _check(got, A, b, c, d, zi, x, out_idx, dtype, name, rev=False):
    """Against the oracle; rev: the model over the flipped row, flipped back."""
    y, zf = got
    w = lambda v: None if v is None else np.asarray(v, np.float64)  # noqa: E731
    xs = np.ascontiguousarray(w(x)[:, ::-1]) if rev else w(x)
    ry, rzf = oracle.lti_state_space(w(A), xs, w(b), w(c), w(d), w(zi), out_idx=out_idx)
    if rev:
        ry = np.ascontiguousarray(ry[:, ::-1])
    D.check(y, ry, f"{name} y", dtype=dtype)
    if zf is not None:
        D.check(zf, rzf, f"{name} zf", dtype=dtype, scale=np.max(np.abs(ry)) if ry.size else None)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("Bn,T", SHAPES)
def test_lti_ss_capi_parity(api, dtype, M, Bn, T):
    for shared in (False, True):
        A, b, c, d, zi, x = _case(dtype, M, Bn, T, shared, D.seed_of("ss", dtype, M, Bn, T, shared))
        name = f"M={M} B={Bn} T={T} shared={shared}"
        _check(_run(api, A, b, c, d, zi, x), A, b, c, d, zi, x, None, dtype, name)
        # b absent (input into state 0), c absent (out_idx), d absent, zi absent
        idx = M - 1
        _check(_run(api, A, None, None, None, None, x, out_idx=idx), A, None, None, None, None, x, idx, dtype,
               name + " e0/out_idx")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("Bn,T", [(1, 1), (2, 17), (3, 3073), (2, 6144), (2, 6145), (2, 12289), (1, 30001)])
def test_lti_ss_capi_reversed(api, dtype, M, Bn, T):
    """phs_lti_ss_rev: the model run backwards in time (zi the state before
    the last sample, zf after the first) is the forward model over the
    flipped row, flipped back; odd lengths take the scalar loads."""
    for shared in (False, True):
        A, b, c, d, zi, x = _case(dtype, M, Bn, T, shared, D.seed_of("ss-rev", dtype, M, Bn, T, shared))
        name = f"rev M={M} B={Bn} T={T} shared={shared}"
        _check(_run(api, A, b, c, d, zi, x, rev=True), A, b, c, d, zi, x, None, dtype, name, rev=True)
        idx = M - 1
        _check(_run(api, A, None, None, None, None, x, out_idx=idx, rev=True), A, None, None, None, None, x, idx,
               dtype, name + " e0/out_idx", rev=True)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("T", [30719, 30720, 30721, 61441])
def test_lti_ss_capi_wide_tile_edges(api, dtype, M, T):
    """Rows on and around the order-2 fp32 plain pass's wide tile (30720
    steps: 15 data waves of 2 x 16 steps per lane) with the normal look-back,
    both time directions: one tile, one tile and one step, three tiles
    (61441 steps, two look-backs per row).  The other orders and fp64 run
    their own tiles over the same rows."""
    for shared in (False, True):
        A, b, c, d, zi, x = _case(dtype, M, 3, T, shared, D.seed_of("ss-wide", dtype, M, T, shared))
        for rev in (False, True):
            name = f"wide M={M} T={T} shared={shared} rev={rev}"
            _check(_run(api, A, b, c, d, zi, x, rev=rev), A, b, c, d, zi, x, None, dtype, name, rev=rev)
        idx = M - 1
        _check(_run(api, A, None, None, None, None, x, out_idx=idx), A, None, None, None, None, x, idx, dtype,
               f"wide M={M} T={T} shared={shared} e0/out_idx")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [2, 4])
def test_lti_ss_capi_reversed_forced_fallback(api, dtype, M):
    lib = api[0]
    # three tiles a row at the order-2 fp32 plain pass's 30720-step tile
    A, b, c, d, zi, x = _case(dtype, M, 3, 2 * 30720 + 5, False, D.seed_of("ss-rev-fallback", dtype, M))
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, A, b, c, d, zi, x, rev=True)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(got, A, b, c, d, zi, x, None, dtype, "rev fallback", rev=True)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [1, 4])
def test_lti_ss_capi_long_rows(api, dtype, M):
    A, b, c, d, zi, x = _case(dtype, M, 2, 1_000_003, False, D.seed_of("ss-long", dtype, M))
    _check(_run(api, A, b, c, d, zi, x), A, b, c, d, zi, x, None, dtype, "long rows")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [2, 3])
def test_lti_ss_capi_forced_fallback(api, dtype, M):
    lib = api[0]
    A, b, c, d, zi, x = _case(dtype, M, 3, 2 * 30720 + 5, False, D.seed_of("ss-fallback", dtype, M))
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, A, b, c, d, zi, x)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(got, A, b, c, d, zi, x, None, dtype, "fallback")


def test_lti_ss_capi_errors(api):
    import torch

    lib, ws, capi = api
    x = torch.zeros((2, 100), device="cuda")
    A = torch.zeros((3, 3), device="cuda")

    def call(dt=0, M=3, out_idx=0, c=None, wsb=ws.numel(), a=A):
        return lib.phs_lti_ss_fwd(dt, M, 2, 100, _p(a), 1, None, 0, _p(c), 1, out_idx, None, 0, None, _p(x), _p(x),
                                  None, _p(ws), wsb, _stream())

    assert call(dt=2) == capi.PHS_ERR_DTYPE
    assert call(M=5) == capi.PHS_ERR_INVALID and call(M=0) == capi.PHS_ERR_INVALID
    assert call(out_idx=3) == capi.PHS_ERR_INVALID and call(out_idx=-1) == capi.PHS_ERR_INVALID
    assert call(a=None) == capi.PHS_ERR_INVALID
    assert call(wsb=lib.phs_lti_ss_workspace_size(0, 3, 2, 100) - 1) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_lti_ss_workspace_size(0, 5, 2, 100) == 0


# ---------------------------------------------------------------- torch API
def _filter(g, order, lead=(), dtype=np.float64):
    """b (order+1 taps), a (order, after the leading 1) with poles of radius < 0.95."""
    A, _, _, _ = _stable_model(g, order, lead)
    a = np.real(np.apply_along_axis(np.poly, -1, np.linalg.eigvals(A).reshape(-1, order))).reshape(
        tuple(lead) + (order + 1,))[..., 1:]
    b = g.standard_normal(tuple(lead) + (order + 1,))
    return b.astype(dtype), a.astype(dtype)


@pytest.mark.parametrize("order", [1, 2, 3, 4])
@pytest.mark.parametrize("form", ["tdf2", "df2"])
@pytest.mark.parametrize("batched", [False, True])
def test_lfilter_orders_take_fused_route(hip, monkeypatch, order, form, batched):
    """lfilter of orders 1, 3, 4 on HIP (philtorch::lfilter_ss) against the
    same call on CPU (the reference's pure-PyTorch route), with zi/zf."""
    import torch

    from philtorch_amd.lti import filtering

    taken = []
    orig = filtering._fused_lfilter_applies
    monkeypatch.setattr(filtering, "_fused_lfilter_applies", lambda *a: taken.append(orig(*a)) or taken[-1])
    g = D.rng(D.seed_of("ss-lfilter", order, form, batched))
    b, a = _filter(g, order, (4,) if batched else ())
    x = g.standard_normal((4, 5000))
    zi = g.standard_normal((4, order))
    tb, ta, tx, tz = (torch.tensor(v) for v in (b, a, x, zi))
    yg, zfg = hip.lti.lfilter(tb.cuda(), ta.cuda(), tx.cuda(), zi=tz.cuda(), form=form, unroll_factor=1)
    # the TDF-II biquad takes the cascade kernel before this route is asked
    assert taken == ([] if (order == 2 and form == "tdf2") else [True])
    yc, zfc = hip.lti.lfilter(tb, ta, tx, zi=tz, form=form, unroll_factor=1)
    D.check(yg.cpu().numpy(), yc.numpy(), "y")
    D.check(zfg.cpu().numpy(), zfc.numpy(), "zf", scale=np.max(np.abs(yc.numpy())))


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_state_space_fused_matches_composed(hip, dtype):
    import torch

    from philtorch_amd.lti import ssm

    g = D.rng(D.seed_of("ss-api", dtype))
    Bn, T, M = 3, 7000, 3
    A, b, c, d = _stable_model(g, M, (Bn,))
    x = g.standard_normal((Bn, T))
    zi = g.standard_normal((Bn, M))
    t = lambda v: torch.tensor(np.asarray(v).astype(dtype), device="cuda")  # noqa: E731
    cases = [
        dict(A=t(A), B=t(b), C=t(c), D=t(d), zi=t(zi)),
        dict(A=t(A[0]), B=t(b[0]), C=t(c[0]), D=t(d[:1]), zi=t(zi[0])),
        dict(A=t(A), B=None, C=None, D=t(d[0]), zi=None, out_idx=1),
        dict(A=t(A[0]), B=t(b), C=t(c[0]), D=None, zi=t(zi)),
    ]
    for kw in cases:
        out_idx = kw.pop("out_idx", None)
        assert ssm._fused_ss_applies(kw["A"], t(x), kw["B"], kw["C"], kw["D"], kw["zi"], 1, out_idx)
        got = hip.lti.state_space(x=t(x), unroll_factor=1, out_idx=out_idx, **kw)
        zi_full = None if kw["zi"] is None else kw["zi"].expand(Bn, M)
        ref = ssm._state_space(kw["A"], t(x), kw["B"], kw["C"], kw["D"], zi_full, 1, out_idx, fused=False)
        got = got if isinstance(got, tuple) else (got,)
        ref = ref if isinstance(ref, tuple) else (ref,)
        for gv, rv in zip(got, ref):
            D.check(gv.cpu().numpy(), rv.cpu().numpy(), f"{sorted(kw)} {out_idx}", dtype=dtype,
                    scale=np.max(np.abs(ref[0].cpu().numpy())))


def test_state_space_fused_gradients(hip):
    import torch

    g = D.rng(D.seed_of("ss-grad"))
    Bn, T, M = 2, 25, 3
    A, b, c, d = _stable_model(g, M, (Bn,))
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=True)  # noqa: E731
    args = (t(A), t(b), t(c), t(d), t(g.standard_normal((Bn, M))), t(g.standard_normal((Bn, T))))
    # the op itself (lti.state_space takes the composed route when a gradient is wanted)
    f = lambda A_, b_, c_, d_, z_, x_: torch.ops.philtorch.lti_ss(A_, b_, c_, d_, z_, x_, 0)  # noqa: E731
    assert torch.autograd.gradcheck(f, args)
    assert torch.autograd.gradgradcheck(f, args)
    assert torch.autograd.gradcheck(lambda *a: hip.lti.state_space(a[0], a[5], a[1], a[2], a[3], zi=a[4],
                                                                   unroll_factor=1), args)
    bf, af = (torch.tensor(v, device="cuda", requires_grad=True) for v in _filter(g, 4, (Bn,)))
    xf = args[-1]
    assert torch.autograd.gradcheck(lambda b_, a_, x_: hip.lti.lfilter(b_, a_, x_, unroll_factor=1), (bf, af, xf))


def test_state_space_route_choice(hip):
    import torch

    from philtorch_amd.lti import ssm

    x = torch.randn(3, 50, device="cuda")
    A = torch.randn(3, 3, device="cuda")
    v = torch.randn(3, device="cuda")
    assert ssm._fused_ss_applies(A, x, v, v, None, None, 1, None)
    assert not ssm._fused_ss_applies(A, x, v, v, None, None, 7, None)  # blocked PyTorch route requested
    assert not ssm._fused_ss_applies(A, x, v, None, None, None, 1, None)  # all states out
    assert not ssm._fused_ss_applies(A, x.unsqueeze(-1), v, v, None, None, 1, None)  # features
    assert not ssm._fused_ss_applies(torch.randn(5, 5, device="cuda"), x, None, None, None, None, 1, 0)
    assert not ssm._fused_ss_applies(A, x, v, v, torch.randn(2, device="cuda"), None, 1, None)
    assert not ssm._fused_ss_applies(A, x.cpu(), v, v, None, None, 1, None)
    assert not ssm._fused_ss_applies(A.double(), x, v, v, None, None, 1, None)
    assert ssm._fused_ss_applies(A, x.requires_grad_(), v, v, None, None, 1, None)  # grad_x by the adjoint
    # coefficient gradients: the fused backward (philtorch::lti_ss_backward)
    assert ssm._fused_ss_applies(A.requires_grad_(), x, v, v, None, None, 1, None)
    with torch.no_grad():
        assert ssm._fused_ss_applies(A, x, v, v, None, None, 1, None)


def test_lti_ss_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("ss-opcheck"))
    A, b, c, d = _stable_model(g, 3, (2,))
    t = lambda v: torch.tensor(np.asarray(v, np.float32), device="cuda")  # noqa: E731
    x = t(g.standard_normal((2, 700)))
    torch.library.opcheck(torch.ops.philtorch.lti_ss.default, (t(A), t(b), t(c), t(d), t(g.standard_normal((2, 3))), x, 0))
    torch.library.opcheck(torch.ops.philtorch.lti_ss.default, (t(A[0]), None, None, None, None, x, 2))


# ---------------------------------------------------------------- lfilter from b and a
def _companion_model(b, a, form):
    """The companion-form state space philtorch's lfilter builds
    (lti/filtering.py:273-333), in numpy: (A, B, C, D, out_idx)."""
    M = max(b.shape[-1] - 1, a.shape[-1])
    b = np.concatenate([b, np.zeros(b.shape[:-1] + (M + 1 - b.shape[-1],))], -1)
    a = np.concatenate([a, np.zeros(a.shape[:-1] + (M - a.shape[-1],))], -1)
    comp = np.zeros(a.shape[:-1] + (M, M))
    comp[..., 0, :] = -a
    comp[..., np.arange(1, M), np.arange(M - 1)] = 1.0
    g = b[..., 1:] - b[..., :1] * a
    if form == "tdf2":
        return np.swapaxes(comp, -1, -2), g, None, b[..., 0], 0
    return comp, None, g, b[..., 0], None


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("nb,na", [(2, 1), (1, 2), (3, 1), (4, 3), (5, 4), (2, 4), (5, 2)])
@pytest.mark.parametrize("form", ["tdf2", "df2"])
@pytest.mark.parametrize("rev", [False, True])
def test_lfilter_capi_parity(api, dtype, nb, na, form, rev):
    """phs_lfilter_fwd (companion model built in the kernel from b and a,
    zero-padded to the order) against the oracle's state space of the
    companion model, shared and per row, at tile boundaries and beyond."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(dtype)]
    M = max(nb - 1, na)
    for (Bn, T), shared in (((3, 3073), False), ((2, 1536), True), ((1, 5), False), ((2, 20001), True)):
        g = D.rng(D.seed_of("lfilter-capi", dtype, nb, na, form, Bn, T, shared))
        lead = () if shared else (Bn,)
        _, aa = _filter(g, na, lead)  # stable denominator of order na
        bb = g.standard_normal(lead + (nb,))
        x = g.standard_normal((Bn, T)).astype(dtype)
        zi = g.standard_normal((Bn, M)).astype(dtype)
        bb, aa = bb.astype(dtype), aa.astype(dtype)
        tb, ta, tx, tz = _dev(bb), _dev(aa), _dev(x), _dev(zi)
        y = torch.full_like(tx, float("nan"))
        zf = torch.full((Bn, M), float("nan"), dtype=tx.dtype, device="cuda")
        need = lib.phs_lti_ss_workspace_size(dt, M, Bn, T)
        fn = lib.phs_lfilter_rev if rev else lib.phs_lfilter_fwd
        rc = fn(dt, Bn, T, _p(tb), nb, _p(ta), na, int(shared), 0 if form == "tdf2" else 1, _p(tz), _p(tx), _p(y),
                _p(zf), _p(ws), need, _stream())
        assert rc == capi.PHS_OK, lib.phs_error_string(rc)
        torch.cuda.synchronize()
        A, Bv, Cv, Dv, idx = _companion_model(np.asarray(bb, np.float64), np.asarray(aa, np.float64), form)
        xs = np.asarray(x, np.float64)
        ry, rzf = oracle.lti_state_space(A, np.ascontiguousarray(xs[:, ::-1]) if rev else xs, Bv, Cv, Dv,
                                         np.asarray(zi, np.float64), out_idx=idx)
        if rev:
            ry = np.ascontiguousarray(ry[:, ::-1])
        name = f"nb={nb} na={na} {form} rev={rev} B={Bn} T={T} shared={shared}"
        D.check(y.cpu().numpy(), ry, name + " y", dtype=dtype)
        D.check(zf.cpu().numpy(), rzf, name + " zf", dtype=dtype, scale=np.max(np.abs(ry)))


def test_lfilter_companion_model_matches_scipy():
    """The companion model of the test above, through the oracle, is
    scipy.signal.lfilter in TDF-II (zero and nonzero initial conditions) and
    in DF-II (zero initial conditions)."""
    import scipy.signal as sg

    g = D.rng(D.seed_of("lfilter-companion"))
    b, a = _filter(g, 4)
    b = b[:3]
    x = g.standard_normal((1, 700))
    zi = g.standard_normal((1, 4))
    for form in ("tdf2", "df2"):
        A, Bv, Cv, Dv, idx = _companion_model(b, a, form)
        y, _ = oracle.lti_state_space(A, x, Bv, Cv, Dv, None, out_idx=idx)
        D.check(y[0], sg.lfilter(b, np.r_[1.0, a], x[0]), form)
    A, Bv, Cv, Dv, idx = _companion_model(b, a, "tdf2")
    y, zf = oracle.lti_state_space(A, x, Bv, Cv, Dv, zi, out_idx=idx)
    ry, rzf = sg.lfilter(b, np.r_[1.0, a], x[0], zi=zi[0])
    D.check(y[0], ry, "tdf2 zi")
    D.check(zf[0], rzf, "tdf2 zf", scale=np.max(np.abs(ry)))


def test_lfilter_ss_op_gradients_and_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("lfilter-ss-grad"))
    b, a = (torch.tensor(v, device="cuda", requires_grad=True) for v in _filter(g, 3, (2,)))
    x = torch.tensor(g.standard_normal((2, 30)), device="cuda", requires_grad=True)
    zi = torch.tensor(g.standard_normal((2, 3)), device="cuda", requires_grad=True)
    for form in (0, 1):
        f = lambda b_, a_, z_, x_: torch.ops.philtorch.lfilter_ss(b_, a_, z_, x_, form)  # noqa: E731
        assert torch.autograd.gradcheck(f, (b, a, zi, x))
        assert torch.autograd.gradgradcheck(f, (b, a, zi, x))
    t = lambda v: torch.tensor(np.asarray(v, np.float32), device="cuda")  # noqa: E731
    bf, af = _filter(g, 4)
    torch.library.opcheck(torch.ops.philtorch.lfilter_ss.default, (t(bf), t(af), None, t(g.standard_normal((2, 500))), 0))
    torch.library.opcheck(torch.ops.philtorch.lfilter_ss.default,
                          (t(bf[:2]), t(af), t(g.standard_normal((2, 4))), t(g.standard_normal((2, 500))), 1))


# ---------------------------------------------------------------- adjoint (grad w.r.t. x and zi)
@pytest.mark.parametrize("order", [1, 3, 4])
@pytest.mark.parametrize("form", ["tdf2", "df2"])
def test_lfilter_signal_gradient_takes_adjoint_pass(hip, monkeypatch, order, form):
    """lfilter with only x and zi requiring grad runs the fused route forward
    and its adjoint (the other companion form, reversed in time) backward;
    gradients against the CPU (reference) route's autograd."""
    import torch

    from philtorch_amd.lti import filtering

    taken = []
    orig = filtering._fused_lfilter_applies
    monkeypatch.setattr(filtering, "_fused_lfilter_applies", lambda *a: taken.append(orig(*a)) or taken[-1])
    g = D.rng(D.seed_of("ss-adjoint", order, form))
    b, a = _filter(g, order, (3,))
    x = g.standard_normal((3, 4000))
    zi = g.standard_normal((3, order))
    gy = g.standard_normal((3, 4000))
    gzf = g.standard_normal((3, order))
    res = []
    for dev in ("cuda", "cpu"):
        tx = torch.tensor(x, device=dev, requires_grad=True)
        tz = torch.tensor(zi, device=dev, requires_grad=True)
        y, zf = hip.lti.lfilter(torch.tensor(b, device=dev), torch.tensor(a, device=dev), tx, zi=tz, form=form,
                                unroll_factor=1)
        ((y * torch.tensor(gy, device=dev)).sum() + (zf * torch.tensor(gzf, device=dev)).sum()).backward()
        res.append((tx.grad.cpu().numpy(), tz.grad.cpu().numpy()))
    assert taken[0] is True
    D.check(res[0][0], res[1][0], "grad_x")
    D.check(res[0][1], res[1][1], "grad_zi", scale=np.max(np.abs(res[1][0])))


def test_adjoint_passes_gradcheck(hip):
    import torch

    g = D.rng(D.seed_of("ss-adjoint-gradcheck"))
    Bn, T = 2, 25
    A, b, c, d = _stable_model(g, 3, (Bn,))
    t = lambda v, rg=False: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=rg)  # noqa: E731
    x, zi = t(g.standard_normal((Bn, T)), True), t(g.standard_normal((Bn, 3)), True)
    f = lambda z_, x_: torch.ops.philtorch.lti_ss(t(A), t(b), t(c), t(d), z_, x_, 0)  # noqa: E731
    assert torch.autograd.gradcheck(f, (zi, x))
    assert torch.autograd.gradgradcheck(f, (zi, x))
    f2 = lambda z_, x_: torch.ops.philtorch.lti_ss(t(A[0]), None, None, None, z_, x_, 2)  # noqa: E731
    assert torch.autograd.gradcheck(f2, (zi, x))
    bf, af = (t(v) for v in _filter(g, 4, (Bn,)))
    z4 = t(g.standard_normal((Bn, 4)), True)
    for form in (0, 1):
        f3 = lambda z_, x_: torch.ops.philtorch.lfilter_ss(bf, af, z_, x_, form)  # noqa: E731
        assert torch.autograd.gradcheck(f3, (z4, x))
        assert torch.autograd.gradgradcheck(f3, (z4, x))


def test_reversed_ops_gradients_and_opcheck(hip):
    """lti_ss and lfilter_ss with reverse=True: values are the forward op
    over the flipped row, flipped back; gradients (the adjoint pass forward
    in time, or the composite when a coefficient needs one) pass gradcheck
    and gradgradcheck; opcheck's schema and fake-tensor checks."""
    import torch

    g = D.rng(D.seed_of("ss-rev-grad"))
    Bn, T = 2, 25
    A, b, c, d = _stable_model(g, 3, (Bn,))
    t = lambda v, rg=False: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=rg)  # noqa: E731
    x, zi = t(g.standard_normal((Bn, T)), True), t(g.standard_normal((Bn, 3)), True)
    y, zf = torch.ops.philtorch.lti_ss(t(A), t(b), t(c), t(d), zi, x, 0, True)
    yr, zfr = torch.ops.philtorch.lti_ss(t(A), t(b), t(c), t(d), zi, x.flip(-1), 0)
    D.check(y.detach().cpu().numpy(), yr.flip(-1).detach().cpu().numpy(), "lti_ss reverse y")
    D.check(zf.detach().cpu().numpy(), zfr.detach().cpu().numpy(), "lti_ss reverse zf")
    f = lambda z_, x_: torch.ops.philtorch.lti_ss(t(A), t(b), t(c), t(d), z_, x_, 0, True)  # noqa: E731
    assert torch.autograd.gradcheck(f, (zi, x))
    assert torch.autograd.gradgradcheck(f, (zi, x))
    Ag, bg = t(A, True), t(b, True)
    fA = lambda A_, b_, x_: torch.ops.philtorch.lti_ss(A_, b_, t(c), t(d), None, x_, 0, True)[0]  # noqa: E731
    assert torch.autograd.gradcheck(fA, (Ag, bg, x))
    bf, af = (t(v) for v in _filter(g, 4, (Bn,)))
    z4 = t(g.standard_normal((Bn, 4)), True)
    for form in (0, 1):
        y, zf = torch.ops.philtorch.lfilter_ss(bf, af, z4, x, form, True)
        yr, zfr = torch.ops.philtorch.lfilter_ss(bf, af, z4, x.flip(-1), form)
        D.check(y.detach().cpu().numpy(), yr.flip(-1).detach().cpu().numpy(), f"lfilter_ss reverse y {form}")
        D.check(zf.detach().cpu().numpy(), zfr.detach().cpu().numpy(), f"lfilter_ss reverse zf {form}")
        f3 = lambda z_, x_: torch.ops.philtorch.lfilter_ss(bf, af, z_, x_, form, True)  # noqa: E731
        assert torch.autograd.gradcheck(f3, (z4, x))
        assert torch.autograd.gradgradcheck(f3, (z4, x))
        bg4, ag4 = t(bf.detach().cpu().numpy(), True), t(af.detach().cpu().numpy(), True)
        f4 = lambda b_, a_, x_: torch.ops.philtorch.lfilter_ss(b_, a_, None, x_, form, True)[0]  # noqa: E731
        assert torch.autograd.gradcheck(f4, (bg4, ag4, x))
    s = lambda v: torch.tensor(np.asarray(v, np.float32), device="cuda")  # noqa: E731
    bf, af = _filter(g, 4)
    torch.library.opcheck(torch.ops.philtorch.lfilter_ss.default,
                          (s(bf), s(af), None, s(g.standard_normal((2, 500))), 0, True))
    torch.library.opcheck(torch.ops.philtorch.lti_ss.default,
                          (s(A[0]), s(b[0]), None, None, s(g.standard_normal((2, 3))), s(g.standard_normal((2, 500))),
                           1, True))



@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", [2, 4])
def test_lti_ss_capi_aggregates_only_multi_window(api, dtype, M):
    """Tiles after a row's first publish aggregates only (testing hook), so
    every look-back folds back to tile 0 through windows of 64 entries: 110
    tiles of 6144 (fp32) or fewer steps per row, both time directions."""
    lib = api[0]
    # 70+ tiles a row at the widest tile (order-2 fp32 plain: 30720 steps)
    A, b, c, d, zi, x = _case(dtype, M, 2, 70 * 30720 + 5, False, D.seed_of("ss-agg-only", dtype, M))
    lib.phs_debug_set_aggregates_only(1)
    try:
        got = _run(api, A, b, c, d, zi, x)
        got_rev = _run(api, A, b, c, d, zi, x, rev=True)
    finally:
        lib.phs_debug_set_aggregates_only(0)
    _check(got, A, b, c, d, zi, x, None, dtype, "aggregates only")
    _check(got_rev, A, b, c, d, zi, x, None, dtype, "aggregates only rev", rev=True)
