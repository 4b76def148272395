"""GPU parity of the fused multi-input multi-output LTI state space
(phs_mimo_ss_fwd / phs_mimo_ss_rev, op philtorch::mimo_ss, the route of
philtorch_amd.lti.state_space for a 3D x or matrix-valued B, C, D).

The C ABI entry points (ctypes, raw device pointers, the caller's stream)
against oracle.lti_state_space_mimo (B x per step, the oracle's lti_recurN,
the shifted state sequence and C h + D x; pinned to scipy.signal.dlsim's
multi-input multi-output simulation in tests/test_oracle.py), evaluated in
fp64 on the GPU's exact inputs.  Orders 1 to 4; 1 to 4 inputs and outputs;
shared and per-row A, B, C, D; D absent; initial and final states; rows
shorter than a lane's chunk, on and around a wave's span (512 fp32 steps,
256 fp64) and a tile (1536 fp32, 768 fp64), of odd length and of a million
steps; both time directions; the forced look-back fallback and
aggregates-only publishing; empty rows.  Through the torch API: every shape
branch of the reference's B, C, D rules that the fused route takes, against
the composed route; gradients (the adjoint pass, the states passes and the
fused sums over time) against the composed route's and by gradcheck, second order
through the composite formula; opcheck.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import _data as D
from tests.test_oracle import _stable_model

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


def _dev(x):
    import torch

    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _run(api, A, Bm, Cm, Dm, zi, x, rev=False, want_zf=True):
    """phs_mimo_ss_fwd (phs_mimo_ss_rev) through the C ABI; numpy (y, zf).
    An operand with one axis fewer than its per-row form is shared."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    Bn, T, F = x.shape
    M, P = A.shape[-1], Cm.shape[-2]
    need = lib.phs_mimo_ss_workspace_size(dt, M, Bn, T)
    assert 0 < need <= ws.numel()
    tA, tB, tC, tD, tz, tx = (_dev(v) for v in (A, Bm, Cm, Dm, zi, x))
    y = torch.full((Bn, T, P), float("nan"), dtype=tx.dtype, device="cuda")
    zf = torch.full((Bn, M), float("nan"), dtype=tx.dtype, device="cuda") if want_zf else None
    shared = ((A.ndim == 2) * capi.PHS_MIMO_A_SHARED | (Bm.ndim == 2) * capi.PHS_MIMO_B_SHARED |
              (Cm.ndim == 2) * capi.PHS_MIMO_C_SHARED | (Dm is not None and Dm.ndim == 2) * capi.PHS_MIMO_D_SHARED)
    fn = lib.phs_mimo_ss_rev if rev else lib.phs_mimo_ss_fwd
    print(f"mimo_ss capi M={M} F={F} P={P} B={Bn} T={T} rev={rev} shared={shared}", flush=True)
    rc = fn(dt, M, F, P, Bn, T, _p(tA), _p(tB), _p(tC), _p(tD), shared, _p(tz), _p(tx), _p(y), _p(zf), _p(ws), need,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    return y.cpu().numpy(), None if zf is None else zf.cpu().numpy()


def _well_conditioned_A(g, M, lead):
    """A stable dense A (_stable_model) whose eigenbasis is well conditioned
    (cond(A) < 1e3 in every row): a random basis occasionally comes out
    nearly singular, and then any reordering of the sum, the scan's included,
    moves fp64 results by 1e-9 of their range."""
    for _ in range(50):
        A = _stable_model(g, M, lead)[0]
        if np.all(np.linalg.cond(A.reshape((-1, M, M))) < 1e3):
            return A
    raise AssertionError("no well-conditioned model drawn")


def _case(dtype, M, F, P, Bn, T, shared, seed, with_d=True):
    g = D.rng(seed)
    lead = () if shared else (Bn,)
    A = _well_conditioned_A(g, M, lead)
    Bm = g.standard_normal(lead + (M, F)) / np.sqrt(F)
    Cm = g.standard_normal(lead + (P, M))
    Dm = g.standard_normal(lead + (P, F)) if with_d else None
    x = g.standard_normal((Bn, T, F))
    zi = g.standard_normal((Bn, M))
    cast = lambda v: None if v is None else np.asarray(v).astype(dtype)  # noqa: E731
    return [cast(v) for v in (A, Bm, Cm, Dm, zi, x)]


def _check(got, A, Bm, Cm, Dm, zi, x, dtype, name, rev=False):
    """Against the oracle; rev: the model over the time-flipped row, flipped back."""
    y, zf = got
    w = lambda v: None if v is None else np.asarray(v, np.float64)  # noqa: E731
    xs = np.ascontiguousarray(w(x)[:, ::-1]) if rev else w(x)
    ry, rzf = oracle.lti_state_space_mimo(w(A), xs, w(Bm), w(Cm), w(Dm), w(zi))
    if rev:
        ry = np.ascontiguousarray(ry[:, ::-1])
    D.check(y, ry, f"{name} y", dtype=dtype)
    if zf is not None:
        D.check(zf, rzf, f"{name} zf", dtype=dtype, scale=np.max(np.abs(ry)) if ry.size else None)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("F,P", WIDTHS)
@pytest.mark.parametrize("Bn,T", SHAPES)
def test_mimo_ss_capi_parity(api, dtype, M, F, P, Bn, T):
    seed = D.seed_of("mimo", np.dtype(dtype).name, M, F, P, Bn, T)
    args = _case(dtype, M, F, P, Bn, T, shared=(T % 2 == 1), seed=seed, with_d=(Bn != 3))
    _check(_run(api, *args), *args, dtype, f"M={M} F={F} P={P} B={Bn} T={T}")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M", ORDERS)
@pytest.mark.parametrize("Bn,T", [(2, 7), (3, 1536), (2, 1537), (2, 20001)])
def test_mimo_ss_capi_reversed(api, dtype, M, Bn, T):
    args = _case(dtype, M, 3, 2, Bn, T, shared=False, seed=D.seed_of("mimo-rev", np.dtype(dtype).name, M, Bn, T))
    _check(_run(api, *args, rev=True), *args, dtype, f"rev M={M} B={Bn} T={T}", rev=True)


@pytest.mark.parametrize("M", [2, 4])
def test_mimo_ss_capi_long_rows(api, M):
    """A million steps per row: hundreds of tiles resolved by the look-back."""
    for dtype in FLOATS:
        args = _case(dtype, M, 2, 3, 2, 1 << 20, shared=True, seed=D.seed_of("mimo-long", M, np.dtype(dtype).name))
        _check(_run(api, *args), *args, dtype, f"long M={M} {np.dtype(dtype).name}")


@pytest.mark.parametrize("M", [1, 3])
def test_mimo_ss_capi_forced_fallback_and_aggregates_only(api, M):
    """The look-back's bounded-wait fallback (each tile folds its row's
    inputs itself) and aggregates-only publishing give the same results."""
    lib = api[0]
    for dtype in FLOATS:
        args = _case(dtype, M, 4, 3, 3, 9001, shared=False, seed=D.seed_of("mimo-fb", M, np.dtype(dtype).name))
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


def test_mimo_ss_capi_empty_rows_and_no_zf(api):
    """T = 0 writes zi as the final state (zeros without zi); zf NULL is
    skipped; the zero-state response without zi."""
    A, Bm, Cm, Dm, zi, x = _case(np.float64, 3, 2, 2, 2, 0, shared=True, seed=5)
    y, zf = _run(api, A, Bm, Cm, Dm, zi, x)
    assert y.shape == (2, 0, 2)
    np.testing.assert_array_equal(zf, zi)
    _, zf0 = _run(api, A, Bm, Cm, Dm, None, x)
    np.testing.assert_array_equal(zf0, np.zeros_like(zi))
    A, Bm, Cm, Dm, zi, x = _case(np.float32, 2, 3, 4, 2, 3000, shared=False, seed=6)
    got = _run(api, A, Bm, Cm, Dm, None, x, want_zf=False)
    assert got[1] is None
    _check(got, A, Bm, Cm, Dm, None, x, np.float32, "no zi, no zf")


def test_mimo_ss_capi_errors(api):
    lib, ws, capi = api
    d = ctypes.c_void_p(ws.data_ptr())

    def call(M=2, F=2, P=2, T=100, wsb=1 << 20, a=d):
        return lib.phs_mimo_ss_fwd(0, M, F, P, 2, T, a, d, d, None, 0, None, d, d, None, d, wsb, None)

    assert call(F=5) == capi.PHS_ERR_INVALID and call(P=0) == capi.PHS_ERR_INVALID
    assert call(M=5) == capi.PHS_ERR_INVALID and call(a=None) == capi.PHS_ERR_INVALID
    assert call(wsb=16) == capi.PHS_ERR_WORKSPACE


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("M,F,P", [(1, 1, 1), (4, 4, 4), (3, 2, 1), (2, 4, 3)])
@pytest.mark.parametrize("Bn,T", [(1, 1), (3, 700), (2, 16384), (2, 16385), (3, 100003), (1, 200003), (70, 5),
                                  (70001, 3)])
def test_mimo_ss_grad_sums_capi(api, dtype, M, F, P, Bn, T):
    """phs_mimo_ss_grad_sums (the coefficient gradients' sums over time)
    against numpy's einsum in fp64: every product per row and over the rows,
    subsets of the products (those reading all four signals and those
    reading two or three), across its 16384-step blocks, past the unrolled
    sums of a row's 13 blocks and of 70 rows' totals, more rows than a
    grid dimension of 65535 holds; A's product per step
    (PHS_MIMO_A_STEPS, transposed or not) bit-exact against numpy's
    product in the same dtype; the input's gradient B^T lambda + D^T g per
    step (B and D per row, B shared without D, alone or beside the sums)."""
    import torch

    lib, ws, capi = api
    g = D.rng(D.seed_of("grad-sums", np.dtype(dtype).name, M, F, P, Bn, T))
    hl = {n: g.standard_normal((Bn, T, w)).astype(dtype) for n, w in (("lam", M), ("hs", M), ("x", F), ("g", P))}
    dv = {n: _dev(v) for n, v in hl.items()}
    w64 = {n: v.astype(np.float64) for n, v in hl.items()}
    refs = [np.einsum("bti,btj->bij", w64[l], w64[r]) for l, r in (("lam", "hs"), ("lam", "x"), ("g", "hs"), ("g", "x"))]
    dims = [(M, M), (M, F), (P, M), (P, F)]
    dt = capi.DTYPES[np.dtype(dtype)]
    need = lib.phs_mimo_ss_grad_sums_scratch_size(dt, Bn, T)
    assert 0 < need
    scratch = ws if need <= ws.numel() else torch.empty(need, dtype=torch.uint8, device="cuda")
    steps_ref = hl["lam"][..., :, None] * hl["hs"][..., None, :]  # per-step products, rounded once
    # the model's B and D for the input's gradient, per row and shared
    Bm_rows, Dm_rows = g.standard_normal((Bn, M, F)), g.standard_normal((Bn, P, F))
    model = {n: _dev(v.astype(dtype)) for n, v in (("B", Bm_rows), ("D", Dm_rows), ("B1", Bm_rows[:1, :, :]),
                                                       ("D1", Dm_rows[:1, :, :]))}
    # (want, shared, input's gradient: None, "rows" (B, D per row), "shared" (one B, no D))
    cases = ((15, 0, None), (15, 15, None), (9, 1, None), (6, 4, None), (8, 8, None), (3, 2, None), (1, 0, None),
             (1, 16, None), (15, 16 | 32 | 2, None), (11, 16 | 8, None), (15, 0, "rows"), (0, 2 | 8, "shared"),
             (1, 16, "rows"))
    for want, shared, gxm in cases:
        outs = [torch.full(((1 if (shared >> i) & 1 else Bn),) + dims[i], float("nan"), dtype=dv["x"].dtype,
                           device="cuda") if (want >> i) & 1 else None for i in range(4)]
        if shared & 16:
            outs[0] = torch.full((Bn, T, M, M), float("nan"), dtype=dv["x"].dtype, device="cuda")
        gx = torch.full((Bn, T, F), float("nan"), dtype=dv["x"].dtype, device="cuda") if gxm else None
        bm = model["B"] if gxm == "rows" else model["B1"] if gxm else None
        dm = model["D"] if gxm == "rows" else None
        print(f"grad_sums M={M} F={F} P={P} B={Bn} T={T} want={want} shared={shared} gx={gxm}", flush=True)
        rc = lib.phs_mimo_ss_grad_sums(dt, M, F, P, Bn, T, _p(dv["lam"]), _p(dv["hs"]), _p(dv["x"]), _p(dv["g"]),
                                       _p(bm), _p(dm), shared, *(_p(o) for o in outs), _p(gx), _p(scratch), need,
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == capi.PHS_OK, lib.phs_error_string(rc)
        torch.cuda.synchronize()
        if gxm:  # B^T lambda + D^T g per step, from the model as the kernel read it, in fp64
            bref = (Bm_rows if gxm == "rows" else np.broadcast_to(Bm_rows[:1], Bm_rows.shape)).astype(dtype)
            gx_ref = np.einsum("bmf,btm->btf", bref.astype(np.float64), w64["lam"])
            if gxm == "rows":
                gx_ref += np.einsum("bpf,btp->btf", Dm_rows.astype(dtype).astype(np.float64), w64["g"])
            D.check(gx.cpu().numpy(), gx_ref, f"input's gradient {gxm}", dtype=dtype, scale=1.0)
        for i in range(4):
            if outs[i] is None:
                continue
            if i == 0 and shared & 16:  # A per step: bit-exact
                ref = np.swapaxes(steps_ref, -1, -2) if shared & 32 else steps_ref
                np.testing.assert_array_equal(outs[0].cpu().numpy(), ref, err_msg=f"A per step shared={shared}")
                continue
            want_i = refs[i].sum(0, keepdims=True) if (shared >> i) & 1 else refs[i]
            # sums of T products: the bound scales with sqrt(T) times the terms' size
            D.check(outs[i].cpu().numpy(), want_i, f"product {i} shared={shared}", dtype=dtype,
                    scale=np.sqrt(Bn * T))


def test_mimo_ss_grad_sums_op_and_empty_rows(hip):
    import torch

    t = lambda *s: torch.randn(*s, device="cuda", dtype=torch.float64)  # noqa: E731
    lam, hs, x, g = t(3, 5000, 2), t(3, 5000, 2), t(3, 5000, 3), t(3, 5000, 4)
    gA, gB, gC, gD = torch.ops.philtorch.mimo_ss_grad_sums(lam, hs, x, g, 0b1010, 15)
    torch.testing.assert_close(gA, torch.einsum("bti,btj->bij", lam, hs))
    torch.testing.assert_close(gB[0], torch.einsum("bti,btj->ij", lam, x))
    torch.testing.assert_close(gC, torch.einsum("bti,btj->bij", g, hs))
    torch.testing.assert_close(gD[0], torch.einsum("bti,btj->ij", g, x))
    none = torch.ops.philtorch.mimo_ss_grad_sums(None, None, x, g, 0, 8)
    assert [v.numel() for v in none[:3]] == [0, 0, 0]
    torch.testing.assert_close(none[3], torch.einsum("bti,btj->bij", g, x))
    e = torch.ops.philtorch.mimo_ss_grad_sums(None, None, x[:, :0], g[:, :0], 8, 8)
    assert e[3].shape == (1, 4, 3) and e[3].abs().sum() == 0
    # the input's gradient beside the sums: B per row, D shared (bit 3)
    Bm, Dm = t(3, 2, 3), t(4, 3)
    *_, gx = torch.ops.philtorch.mimo_ss_grad_sums(lam, hs, x, g, 0b1000, 31, Bm, Dm)
    torch.testing.assert_close(gx, torch.einsum("bmf,btm->btf", Bm, lam) + torch.einsum("pf,btp->btf", Dm, g))
    f = lambda v: v.float()  # noqa: E731
    torch.library.opcheck(torch.ops.philtorch.mimo_ss_grad_sums.default, (f(lam), f(hs), f(x), f(g), 5, 15))
    torch.library.opcheck(torch.ops.philtorch.mimo_ss_grad_sums.default,
                          (f(lam), f(hs), f(x), f(g), 8, 31, f(Bm), f(Dm)))


# ---------------------------------------------------------------- torch API
def _api_cases(batch, M):
    from tests.test_host import _mimo_shape_cases

    return _mimo_shape_cases(batch, M)


@pytest.mark.parametrize("dtype", ["float32", "float64"])
@pytest.mark.parametrize("case", range(12))
def test_state_space_mimo_route_matches_composed(hip, monkeypatch, dtype, case):
    """lti.state_space on every shape branch the fused multi-output route
    takes: the route runs philtorch::mimo_ss (and not the single-output op),
    and y, zf agree with the composed route (B x, the native scan, the state
    shift, C h + D x) on the same device."""
    import torch

    from philtorch_amd.lti import ssm

    batch, N, M = 4, 5000, 3
    F, bs, cs, ds, out_idx = _api_cases(batch, M)[case]
    dt = getattr(torch, dtype)
    g = torch.Generator().manual_seed(2000 + case)
    rnd = lambda *s: torch.randn(tuple(s), generator=g, dtype=torch.float64).to(dt).cuda()  # noqa: E731
    A = torch.tensor(_well_conditioned_A(D.rng(case), M, ()), dtype=dt).cuda()
    x = rnd(batch, N) if F is None else rnd(batch, N, F)
    B = None if bs is None else rnd(*bs)
    C = None if cs is None else rnd(*cs)
    Dm = None if ds is None else rnd(*ds)
    zi = rnd(batch, M)
    calls = []
    real = torch.ops.philtorch.mimo_ss

    class Spy:
        def __call__(self, *a, **k):
            calls.append(a[0].shape)
            return real(*a, **k)

    monkeypatch.setattr(torch.ops.philtorch, "mimo_ss", Spy())
    print(f"state_space mimo case {case} {dtype}", flush=True)
    y, zf = hip.lti.state_space(A, x, B, C, Dm, zi=zi, unroll_factor=1, out_idx=out_idx)
    assert calls, "the fused multi-output route was not taken"
    ref, rzf = ssm._state_space(A, x, B, C, Dm, zi, 1, out_idx, fused=False)
    assert y.shape == ref.shape
    D.check(y.double().cpu().numpy(), ref.double().cpu().numpy(), f"case {case} y", dtype=np.dtype(dtype))
    D.check(zf.double().cpu().numpy(), rzf.double().cpu().numpy(), f"case {case} zf", dtype=np.dtype(dtype),
            scale=float(ref.abs().max()))
    y2 = hip.lti.state_space(A, x, B, C, Dm, unroll_factor=1, out_idx=out_idx)  # no zi: no zf
    ref2 = ssm._state_space(A, x, B, C, Dm, None, 1, out_idx, fused=False)
    D.check(y2.double().cpu().numpy(), ref2.double().cpu().numpy(), f"case {case} y no zi", dtype=np.dtype(dtype))


@pytest.mark.parametrize("shared", [False, True])
def test_mimo_ss_gradients_match_composed_route(hip, shared):
    """Gradients of every input through the fused op (the adjoint pass, the
    two states passes and the per-operand sums over time and rows) against
    the composed route's autograd, fp64, rows over several tiles."""
    import torch

    from philtorch_amd.lti import ssm

    batch, N, M, F, P = 3, 4000, 3, 2, 4
    g = D.rng(D.seed_of("mimo-grad", shared))
    lead = () if shared else (batch,)
    A0 = _well_conditioned_A(g, M, lead)
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=True)  # noqa: E731
    ins = [t(A0), t(g.standard_normal(lead + (M, F))), t(g.standard_normal(lead + (P, M))),
           t(g.standard_normal(lead + (P, F))), t(g.standard_normal((batch, M))), t(g.standard_normal((batch, N, F)))]
    gy = torch.tensor(g.standard_normal((batch, N, P)), device="cuda")
    gzf = torch.tensor(g.standard_normal((batch, M)), device="cuda")
    print(f"mimo grads shared={shared}", flush=True)
    y, zf = torch.ops.philtorch.mimo_ss(*ins)
    got = torch.autograd.grad([y, zf], ins, [gy, gzf])
    ry, rzf = ssm._mimo_composite(*ins)
    ref = torch.autograd.grad([ry, rzf], ins, [gy, gzf])
    for name, a, b in zip("A B C D zi x".split(), got, ref):
        D.check(a.cpu().numpy(), b.cpu().numpy(), f"grad {name}", dtype=np.float64)
    # grad_x alone takes the adjoint pass only
    fixed = [v.detach() for v in ins[:5]]
    (gx,) = torch.autograd.grad([torch.ops.philtorch.mimo_ss(*fixed, ins[5])[0]], [ins[5]], [gy])
    (rgx,) = torch.autograd.grad([ssm._mimo_composite(*fixed, ins[5])[0]], [ins[5]], [gy])
    D.check(gx.cpu().numpy(), rgx.cpu().numpy(), "grad x alone", dtype=np.float64)


def test_mimo_ss_gradcheck_and_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("mimo-gradcheck"))
    batch, N, M, F, P = 2, 40, 2, 3, 2
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=True)  # noqa: E731
    A = t(_well_conditioned_A(g, M, (batch,)))
    Bm, Cm, Dm = t(g.standard_normal((M, F))), t(g.standard_normal((batch, P, M))), t(g.standard_normal((P, F)))
    zi, x = t(g.standard_normal((batch, M))), t(g.standard_normal((batch, N, F)))
    op = torch.ops.philtorch.mimo_ss
    print("mimo gradcheck", flush=True)
    assert torch.autograd.gradcheck(lambda *a: op(*a), (A, Bm, Cm, Dm, zi, x))
    assert torch.autograd.gradcheck(lambda *a: op(*a, True), (A, Bm, Cm, Dm, zi, x))
    assert torch.autograd.gradgradcheck(lambda *a: op(*a)[0], (A, Bm, Cm, Dm, zi, x))
    f32 = lambda v: v.detach().float()  # noqa: E731
    torch.library.opcheck(op.default, tuple(f32(v) for v in (A, Bm, Cm, Dm, zi, x)))
    torch.library.opcheck(op.default, (f32(A[0]), f32(Bm), f32(Cm[0]), None, None, f32(x), True))


def test_state_space_mimo_api_gradcheck(hip):
    """lti.state_space's fused multi-output route through its shape
    handling (B (M, F), C (P, M), scalar D as D I) by gradcheck."""
    import torch

    g = D.rng(D.seed_of("mimo-api-gradcheck"))
    batch, N, M, F = 3, 30, 3, 2  # (F != batch: C (F, M) reads as (P, M))
    t = lambda v: torch.tensor(np.asarray(v, np.float64), device="cuda", requires_grad=True)  # noqa: E731
    A = t(_well_conditioned_A(g, M, ()))
    Bm, Cm, Dm = t(g.standard_normal((M, F))), t(g.standard_normal((F, M))), t(g.standard_normal(()))
    zi, x = t(g.standard_normal((batch, M))), t(g.standard_normal((batch, N, F)))

    def f(A, Bm, Cm, Dm, zi, x):
        return hip.lti.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)

    assert torch.autograd.gradcheck(f, (A, Bm, Cm, Dm, zi, x))
