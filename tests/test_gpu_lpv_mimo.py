"""GPU parity of the fused multi-input multi-output LPV state space
(phs_lpv_mimo_ss, op philtorch::lpv_mimo_ss, the route of
philtorch_amd.lpv.state_space for a 3D x or matrix-valued B, C, D constant in
time).

The C ABI entry point (ctypes, raw device pointers, the caller's stream)
against oracle.lpv_state_space_mimo (B x per step, the oracle's recurN, the
shifted state sequence and C h + D x; pinned to the per-step loop, the LTI
form and the single-input form in tests/test_oracle.py), evaluated in fp64 on
the GPU's exact inputs.  Orders 1 to 4; 1 to 4 inputs and outputs; A per row
and shared, read as it lies or transposed; B, C, D per row and shared; D
absent; initial and final states; rows shorter than a lane's chunk, on and
around a wave's span and a tile, of odd length and of half a million steps;
both time directions; the forced look-back fallback and aggregates-only
publishing; empty rows.  Through the torch API: every shape branch of the
reference's LPV B, C, D rules that the fused route takes, against the
composed route; gradients of every input against the composed route's
autograd and by gradcheck, second order through the composite formula;
opcheck.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import _data as D
from tests.test_gpu_mimo import _dev, _p

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (2, 7), (2, 255), (3, 512), (2, 769), (3, 1536), (2, 1537), (2, 20001)]
FLOATS = [np.float32, np.float64]
ORDERS = [1, 2, 3, 4]
WIDTHS = [(1, 2), (3, 4), (4, 1), (2, 2)]


@pytest.fixture(scope="module")
def api(hip):
    import torch

    from tests import capi

    lib = capi.load()
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    yield lib, ws, capi
    lib.phs_debug_set_spin_limit(0)
    lib.phs_debug_set_aggregates_only(0)


def _contractive_A(g, lead, T, M):
    """A[t] with spectral norm below 0.95 at every step (the product of any
    run of steps contracts, so fp32 rounding does not grow along the row)."""
    A = g.standard_normal(lead + (T, M, M))
    nrm = np.linalg.norm(A, ord=2, axis=(-2, -1))[..., None, None]
    return 0.95 * A / np.maximum(nrm, 1e-12) * g.uniform(0.5, 1.0, lead + (T, 1, 1))


def _run(api, A, Bm, Cm, Dm, zi, x, rev=False, trans=False, want_zf=True):
    """phs_lpv_mimo_ss through the C ABI; numpy (y, zf).  A shared when 3D;
    B, C, D shared when 2D."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    Bn, T, F = x.shape
    M, P = A.shape[-1], Cm.shape[-2]
    need = lib.phs_lpv_mimo_ss_workspace_size(dt, M, Bn, T)
    assert 0 < need <= ws.numel()
    tA, tB, tC, tD, tz, tx = (_dev(v) for v in (A, Bm, Cm, Dm, zi, x))
    y = torch.full((Bn, T, P), float("nan"), dtype=tx.dtype, device="cuda")
    zf = torch.full((Bn, M), float("nan"), dtype=tx.dtype, device="cuda") if want_zf else None
    a_flags = (A.ndim == 3) * capi.PHS_LPV_A_SHARED | trans * capi.PHS_LPV_A_TRANSPOSED
    shared = ((Bm.ndim == 2) * capi.PHS_MIMO_B_SHARED | (Cm.ndim == 2) * capi.PHS_MIMO_C_SHARED |
              (Dm is not None and Dm.ndim == 2) * capi.PHS_MIMO_D_SHARED)
    print(f"lpv_mimo_ss capi M={M} F={F} P={P} B={Bn} T={T} rev={rev} trans={trans} A_flags={a_flags} "
          f"shared={shared}", flush=True)
    rc = lib.phs_lpv_mimo_ss(dt, M, F, P, Bn, T, _p(tA), a_flags, _p(tB), _p(tC), _p(tD), shared, _p(tz), _p(tx),
                             _p(y), _p(zf), int(rev), _p(ws), need,
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    return y.cpu().numpy(), None if zf is None else zf.cpu().numpy()


def _case(dtype, M, F, P, Bn, T, shared, seed, with_d=True):
    g = D.rng(seed)
    lead = () if shared else (Bn,)
    A = _contractive_A(g, () if shared else (Bn,), T, M)
    Bm = g.standard_normal(lead + (M, F)) / np.sqrt(F)
    Cm = g.standard_normal(lead + (P, M))
    Dm = g.standard_normal(lead + (P, F)) if with_d else None
    x = g.standard_normal((Bn, T, F))
    zi = g.standard_normal((Bn, M))
    cast = lambda v: None if v is None else np.asarray(v).astype(dtype)  # noqa: E731
    return [cast(v) for v in (A, Bm, Cm, Dm, zi, x)]


def _check(got, A, Bm, Cm, Dm, zi, x, dtype, name, rev=False, trans=False):
    """Against the oracle; rev: the model over the time-flipped row (A
    flipped along time too), flipped back; trans: A[t]^T."""
    y, zf = got
    w = lambda v: None if v is None else np.asarray(v, np.float64)  # noqa: E731
    Aw = w(A)
    if trans:
        Aw = np.swapaxes(Aw, -1, -2)
    xs = w(x)
    if rev:
        Aw, xs = np.flip(Aw, axis=-3), xs[:, ::-1]
    ry, rzf = oracle.lpv_state_space_mimo(np.ascontiguousarray(Aw), np.ascontiguousarray(xs), w(Bm), w(Cm), w(Dm),
                                          w(zi))
    if rev:
        ry = np.ascontiguousarray(ry[:, ::-1])
    D.check(y, ry, f"{name} y", dtype=dtype)
    if zf is not None:
        D.check(zf, rzf, f"{name} zf", dtype=dtype, scale=np.max(np.abs(ry)) if ry.size else None)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("F,P", WIDTHS)
@pytest.mark.parametrize("Bn,T", SHAPES)
def test_lpv_mimo_ss_capi_parity(api, dtype, M, F, P, Bn, T):
    seed = D.seed_of("lpv-mimo", np.dtype(dtype).name, M, F, P, Bn, T)
    args = _case(dtype, M, F, P, Bn, T, shared=(T % 2 == 1), seed=seed, with_d=(Bn != 3))
    _check(_run(api, *args), *args, dtype, f"M={M} F={F} P={P} B={Bn} T={T}")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("Bn,T", [(2, 7), (3, 1536), (2, 1537), (2, 20001)])
@pytest.mark.parametrize("rev,trans", [(True, False), (False, True), (True, True)])
def test_lpv_mimo_ss_capi_reversed_and_transposed(api, dtype, M, Bn, T, rev, trans):
    args = _case(dtype, M, 3, 2, Bn, T, shared=False,
                 seed=D.seed_of("lpv-mimo-rev", np.dtype(dtype).name, M, Bn, T, rev, trans))
    _check(_run(api, *args, rev=rev, trans=trans), *args, dtype, f"rev={rev} trans={trans} M={M} B={Bn} T={T}",
           rev=rev, trans=trans)


@pytest.mark.parametrize("M", [2, 4])
def test_lpv_mimo_ss_capi_long_rows(api, M):
    """Half a million steps per row: hundreds of tiles resolved by the
    look-back."""
    for dtype in FLOATS:
        args = _case(dtype, M, 2, 3, 2, 1 << 19, shared=True,
                     seed=D.seed_of("lpv-mimo-long", M, np.dtype(dtype).name))
        _check(_run(api, *args), *args, dtype, f"long M={M} {np.dtype(dtype).name}")


@pytest.mark.parametrize("M", [1, 3])
def test_lpv_mimo_ss_capi_forced_fallback_and_aggregates_only(api, M):
    lib = api[0]
    for dtype in FLOATS:
        args = _case(dtype, M, 4, 3, 3, 9001, shared=False,
                     seed=D.seed_of("lpv-mimo-fb", M, np.dtype(dtype).name))
        lib.phs_debug_set_spin_limit(1)
        try:
            _check(_run(api, *args), *args, dtype, f"fallback M={M}")
            _check(_run(api, *args, rev=True), *args, dtype, f"fallback rev M={M}", rev=True)
        finally:
            lib.phs_debug_set_spin_limit(0)
        lib.phs_debug_set_aggregates_only(1)
        try:
            _check(_run(api, *args), *args, dtype, f"aggregates-only M={M}")
        finally:
            lib.phs_debug_set_aggregates_only(0)


def test_lpv_mimo_ss_capi_empty_rows_and_errors(api):
    lib, ws, capi = api
    A, Bm, Cm, Dm, zi, x = _case(np.float64, 3, 2, 2, 2, 0, shared=True, seed=7)
    y, zf = _run(api, A, Bm, Cm, Dm, zi, x)
    assert y.shape == (2, 0, 2)
    np.testing.assert_array_equal(zf, zi)
    d = ctypes.c_void_p(ws.data_ptr())

    def call(M=2, F=2, P=2, a_flags=0, shared=0, wsb=1 << 20, a=d):
        return lib.phs_lpv_mimo_ss(0, M, F, P, 2, 100, a, a_flags, d, d, None, shared, None, d, d, None, 0, d, wsb,
                                   None)

    assert call(F=5) == capi.PHS_ERR_INVALID and call(P=0) == capi.PHS_ERR_INVALID
    assert call(M=5) == capi.PHS_ERR_INVALID and call(a=None) == capi.PHS_ERR_INVALID
    assert call(a_flags=4) == capi.PHS_ERR_INVALID and call(shared=1) == capi.PHS_ERR_INVALID
    assert call(wsb=16) == capi.PHS_ERR_WORKSPACE


# ---------------------------------------------------------------- torch API
@pytest.mark.parametrize("dtype", ["float32", "float64"])
@pytest.mark.parametrize("case", range(12))
def test_lpv_state_space_mimo_route_matches_composed(hip, monkeypatch, dtype, case):
    """lpv.state_space on every shape branch the fused multi-output route
    takes: the route runs philtorch::lpv_mimo_ss, and y, zf agree with the
    composed route (B x, the native LPV scan, the state shift, C h + D x)."""
    import torch

    from philtorch_amd.lpv import ssm
    from tests.test_host import _lpv_mimo_shape_cases

    batch, N, M, F, P = 5, 3000, 3, 2, 4
    Fx, bs, cs, ds, out_idx = _lpv_mimo_shape_cases(batch, N, M, F, P)[case]
    dt = getattr(torch, dtype)
    g = D.rng(D.seed_of("lpv-mimo-api", case))
    t = lambda v: torch.tensor(np.asarray(v), dtype=dt).cuda()  # noqa: E731
    A = t(_contractive_A(g, (batch,) if case % 2 else (), N, M))
    x = t(g.standard_normal((batch, N) if Fx is None else (batch, N, Fx)))
    B = None if bs is None else t(g.standard_normal(bs))
    C = None if cs is None else t(g.standard_normal(cs))
    Dm = None if ds is None else t(g.standard_normal(ds))
    zi = t(g.standard_normal((batch, M)))
    calls = []
    real = torch.ops.philtorch.lpv_mimo_ss

    class Spy:
        def __call__(self, *a, **k):
            calls.append(a[0].shape)
            return real(*a, **k)

    monkeypatch.setattr(torch.ops.philtorch, "lpv_mimo_ss", Spy())
    print(f"lpv state_space mimo case {case} {dtype}", flush=True)
    y, zf = hip.lpv.state_space(A, x, B, C, Dm, zi=zi, unroll_factor=1, out_idx=out_idx)
    assert calls, "the fused multi-output route was not taken"
    monkeypatch.setattr(ssm, "_lpv_mimo_applies", lambda *a, **k: False)
    ref, rzf = hip.lpv.state_space(A, x, B, C, Dm, zi=zi, unroll_factor=1, out_idx=out_idx)
    assert len(calls) == 1
    assert y.shape == ref.shape
    D.check(y.double().cpu().numpy(), ref.double().cpu().numpy(), f"case {case} y", dtype=np.dtype(dtype))
    D.check(zf.double().cpu().numpy(), rzf.double().cpu().numpy(), f"case {case} zf", dtype=np.dtype(dtype),
            scale=float(ref.abs().max()))


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("trans", [False, True])
def test_lpv_mimo_ss_gradients_match_composed_route(hip, shared, trans):
    """Gradients of every input through the fused op (the adjoint pass, the
    two states passes, the per-step products for A and the sums over time
    for B, C, D) against the composed route's autograd, fp64, over several
    tiles; A read as it lies and transposed."""
    import torch

    from philtorch_amd.lpv import ssm

    batch, N, M, F, P = 3, 4000, 3, 2, 4
    g = D.rng(D.seed_of("lpv-mimo-grad", shared, trans))
    lead = () if shared else (batch,)
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=True)  # noqa: E731
    ins = [t(_contractive_A(g, lead, N, M)), t(g.standard_normal(lead + (M, F))), t(g.standard_normal(lead + (P, M))),
           t(g.standard_normal(lead + (P, F))), t(g.standard_normal((batch, M))), t(g.standard_normal((batch, N, F)))]
    gy = torch.tensor(g.standard_normal((batch, N, P)), device="cuda")
    gzf = torch.tensor(g.standard_normal((batch, M)), device="cuda")
    print(f"lpv mimo grads shared={shared} trans={trans}", flush=True)
    y, zf = torch.ops.philtorch.lpv_mimo_ss(*ins, False, trans)
    got = torch.autograd.grad([y, zf], ins, [gy, gzf])
    ry, rzf = ssm._lpv_mimo_composite(*ins, transpose_A=trans)
    ref = torch.autograd.grad([ry, rzf], ins, [gy, gzf])
    for name, a, b in zip("A B C D zi x".split(), got, ref):
        D.check(a.cpu().numpy(), b.cpu().numpy(), f"grad {name}", dtype=np.float64)


def test_lpv_mimo_ss_gradcheck_and_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("lpv-mimo-gradcheck"))
    batch, N, M, F, P = 2, 30, 2, 3, 2
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=True)  # noqa: E731
    A = t(_contractive_A(g, (batch,), N, M))
    Bm, Cm, Dm = t(g.standard_normal((M, F))), t(g.standard_normal((batch, P, M))), t(g.standard_normal((P, F)))
    zi, x = t(g.standard_normal((batch, M))), t(g.standard_normal((batch, N, F)))
    op = torch.ops.philtorch.lpv_mimo_ss
    print("lpv mimo gradcheck", flush=True)
    assert torch.autograd.gradcheck(lambda *a: op(*a), (A, Bm, Cm, Dm, zi, x))
    assert torch.autograd.gradcheck(lambda *a: op(*a, True, True), (A, Bm, Cm, Dm, zi, x))
    assert torch.autograd.gradgradcheck(lambda *a: op(*a)[0], (A, Bm, Cm, Dm, zi, x))
    f32 = lambda v: v.detach().float()  # noqa: E731
    torch.library.opcheck(op.default, tuple(f32(v) for v in (A, Bm, Cm, Dm, zi, x)))
    torch.library.opcheck(op.default, (f32(A[0]), f32(Bm), f32(Cm[0]), None, None, f32(x), True, True))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M,F,P", [(1, 2, 3), (2, 2, 2), (2, 3, 1), (3, 1, 1)])
@pytest.mark.parametrize("rev,trans", [(False, False), (True, False), (False, True)])
def test_lpv_mimo_ss_states_op(hip, dtype, M, F, P, rev, trans):
    """philtorch::lpv_mimo_ss_states (phs_lpv_mimo_ss_hs): y and zf bit for
    bit lpv_mimo_ss's, hs bit for bit the states pass the coefficient
    backward would run (the model again with C the identity, no D), across
    spans and tiles; gradcheck of its (y, zf) and opcheck."""
    import torch

    g = D.rng(D.seed_of("lpv-mimo-states", np.dtype(dtype).name, M, F, P, rev, trans))
    Bn, T = 3, 5003
    t = lambda v: torch.tensor(np.ascontiguousarray(v, dtype=dtype), device="cuda")  # noqa: E731
    A = t(_contractive_A(g, (Bn,), T, M))
    Bm, Cm, Dm = t(g.standard_normal((M, F))), t(g.standard_normal((Bn, P, M))), t(g.standard_normal((P, F)))
    zi, x = t(g.standard_normal((Bn, M))), t(g.standard_normal((Bn, T, F)))
    print(f"lpv_mimo_ss_states {np.dtype(dtype).name} M={M} F={F} P={P} rev={rev} trans={trans}", flush=True)
    y0, zf0 = torch.ops.philtorch.lpv_mimo_ss(A, Bm, Cm, Dm, zi, x, rev, trans)
    y1, zf1, hs = torch.ops.philtorch.lpv_mimo_ss_states(A, Bm, Cm, Dm, zi, x, rev, trans)
    eye = torch.eye(M, dtype=x.dtype, device="cuda")
    h_ref, _ = torch.ops.philtorch.lpv_mimo_ss(A, Bm, eye, None, zi, x, rev, trans)
    assert torch.equal(y0, y1) and torch.equal(zf0, zf1) and torch.equal(hs, h_ref)
    if dtype == np.float64:
        small = [v.detach()[:, :40].contiguous() if v.dim() == 3 and v.size(1) == T else v.detach()
                 for v in (A, Bm, Cm, Dm, zi, x)]
        small[0] = small[0][:, :40].contiguous()
        leaves = [v.clone().requires_grad_(True) for v in small]
        f = lambda *a: torch.ops.philtorch.lpv_mimo_ss_states(*a, rev, trans)[:2]  # noqa: E731
        assert torch.autograd.gradcheck(f, tuple(leaves))
        torch.library.opcheck(torch.ops.philtorch.lpv_mimo_ss_states.default, (*small, rev, trans))
