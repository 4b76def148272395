"""GPU parity of the zero-phase filter (phs_filtfilt_fwd, op
philtorch::filtfilt, the fused route of philtorch_amd.lti.filtfilt for
filters of order 1 to 4: two state-space passes, the second in reversed
time, their entry states derived in the kernel).

The C ABI entry point (ctypes, raw device pointers, the caller's stream)
against oracle.filtfilt_ba, which follows the reference's filtfilt step by
step (pad, lfilter_zi, lfilter, flip, lfilter, trim, flip; pinned to
scipy.signal.filtfilt in tests/test_oracle.py), evaluated in fp64 on the GPU's
exact inputs.  Covers orders 1-4 and unequal numerator / denominator lengths,
every pad mode at padlen 0, 9, an intermediate length and the largest
allowed (T - 1); rows shorter than a lane's chunk, on and around a tile
(6144 fp32 or 3072 fp64 steps) and two, of odd length (scalar loads) and of a
million steps; shared and per-row coefficients; the forced look-back fallback
of both passes; a constant row and linearity at the benchmark's C4 size.
Through the torch API: scipy (orders 1-4), the composed route (each pass an
lfilter) at the C4 size, the route choice, and gradients (which take the
fused route too).

The gradients (phs_filtfilt_bwd, op philtorch::filtfilt_backward): grad_x as
J^T grad_y with J the oracle's filtfilt applied to unit impulses (exact, at
small T, every pad mode, padlen 0 to T - 1) and the adjoint identity
<g, F x> = <F^T g, x> with F the oracle at rows of many tiles; grad_b and
grad_a against central differences of the oracle in fp64 (every pad mode,
orders 1-4, shared and per-row filters, b one tap short, rows of one and
two tiles); the forced look-back fallback; the composed route's autograd
(orders 1-4, every pad mode, 1D and 2D x, x, b and a together and apart,
and the C4 size against the composed route in fp64); gradcheck /
gradgradcheck of the op.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import _data as D

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (2, 17), (2, 3071), (3, 3073), (3, 6143), (2, 6144), (2, 6145), (2, 12287), (3, 12288),
          (1, 40000), (2, 30001)]
ORDERS = [1, 2, 3, 4]
FLOATS = [np.float32, np.float64]
MODES = ["constant", "replicate", "reflect", "circular"]


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

    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _run(api, b, a, x, padmode, padlen):
    """phs_filtfilt_fwd through the C ABI; numpy y."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    B, T = x.shape
    need = lib.phs_filtfilt_workspace_size(dt, B, T)
    assert 0 < need <= ws.numel()
    mid = torch.empty(lib.phs_filtfilt_mid_size(dt, B, T), dtype=torch.uint8, device="cuda")
    tb, ta, tx = _dev(b), _dev(a), _dev(x)
    y = torch.full_like(tx, float("nan"))
    print(f"filtfilt capi B={B} T={T} nb={b.shape[-1]} na={a.shape[-1]} {padmode} {padlen}", flush=True)
    rc = lib.phs_filtfilt_fwd(dt, B, T, _p(tb), b.shape[-1], _p(ta), a.shape[-1], int(b.ndim == 1),
                              capi.PADMODES[padmode], padlen, _p(tx), _p(y), _p(mid), _p(ws), need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _case(dtype, B, T, shared, seed, order=2):
    g = D.rng(seed)
    b, a = D.ba_coefs(g, () if shared else (B,), order, dtype, rhi=0.98)
    x = D.normal(g, (B, T), dtype)
    return b, a, x


def _check(y, b, a, x, padmode, padlen, dtype, name):
    f64 = lambda v: np.asarray(v, np.float64)  # noqa: E731
    ref = oracle.filtfilt_ba(f64(b), f64(a), f64(x), padmode=padmode, padlen=padlen)
    D.check(y, ref, name, dtype=dtype)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("B,T", SHAPES)
def test_filtfilt_capi_parity(api, dtype, order, B, T):
    for shared in (False, True):
        b, a, x = _case(dtype, B, T, shared, D.seed_of("filtfilt", dtype, order, B, T, shared), order)
        for mode in MODES:
            for padlen in sorted({0, min(9, T - 1), T // 3, T - 1}):
                y = _run(api, b, a, x, mode, padlen)
                _check(y, b, a, x, mode, padlen, dtype, f"order {order} B={B} T={T} shared={shared} {mode} "
                       f"padlen={padlen}")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_filtfilt_capi_unequal_lengths(api, dtype):
    """Numerator and denominator of different lengths: the order is
    max(nb - 1, na), the shorter one zero-padded (an FIR, an all-pole
    filter and mixed cases)."""
    g = D.rng(D.seed_of("filtfilt-nbna", dtype))
    x = D.normal(g, (3, 7001), dtype)
    for nb, na in ((5, 1), (1, 4), (2, 3), (4, 2), (3, 1), (1, 1), (2, 4)):
        order = max(nb - 1, na)
        bf, af = D.ba_coefs(g, (3,), order, np.float64, rhi=0.98)
        b = g.standard_normal((3, nb)) if nb != order + 1 else bf
        a = af[:, :na] if na == order else D.ba_coefs(g, (3,), na, np.float64, rhi=0.98)[1]
        b, a = b.astype(dtype), a.astype(dtype)
        for mode, padlen in (("replicate", 3 * (order + 1)), ("reflect", 40), ("constant", 0)):
            _check(_run(api, b, a, x, mode, padlen), b, a, x, mode, padlen, dtype, f"nb={nb} na={na} {mode}")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", [2, 4])
def test_filtfilt_capi_long_rows(api, dtype, order):
    b, a, x = _case(dtype, 2, 1_000_003, False, D.seed_of("filtfilt-long", dtype, order), order)
    for mode, padlen in (("replicate", 9), ("reflect", 4097)):
        _check(_run(api, b, a, x, mode, padlen), b, a, x, mode, padlen, dtype, f"long rows {mode}")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", ORDERS)
def test_filtfilt_capi_forced_fallback(api, dtype, order):
    """A one-poll budget makes the tiles of both passes compute their entry
    states from the row's edge and prefix (pass 1) or suffix (pass 2)
    themselves."""
    lib = api[0]
    b, a, x = _case(dtype, 3, 40000, False, D.seed_of("filtfilt-fallback", dtype, order), order)
    lib.phs_debug_set_spin_limit(1)
    try:
        y = _run(api, b, a, x, "replicate", 9)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(y, b, a, x, "replicate", 9, dtype, "fallback")


def _run_bwd(api, b, a, gy, padmode, padlen, spin_limit=0, x=None):
    """phs_filtfilt_bwd through the C ABI (scratch and outputs prefilled with
    NaN bytes: every value must be written before it is read); numpy
    grad_x, or (grad_x, grad_b, grad_a) when x is given."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(gy.dtype)]
    B, T = gy.shape
    coef = x is not None
    M = max(b.shape[-1] - 1, a.shape[-1])
    need = lib.phs_filtfilt_workspace_size(dt, B, T)
    assert 0 < need <= ws.numel()
    sc = torch.full((lib.phs_filtfilt_bwd_scratch_size(dt, M, B, T, padlen, int(coef)),), 255, dtype=torch.uint8,
                    device="cuda")
    tb, ta, tg = _dev(b), _dev(a), _dev(gy)
    tx = _dev(x) if coef else None
    gx = torch.full_like(tg, float("nan"))
    gb = torch.full_like(tb, float("nan")) if coef else None
    ga = torch.full_like(ta, float("nan")) if coef else None
    print(f"filtfilt_bwd capi B={B} T={T} nb={b.shape[-1]} na={a.shape[-1]} {padmode} {padlen} coef={coef}",
          flush=True)
    lib.phs_debug_set_spin_limit(spin_limit)
    try:
        rc = lib.phs_filtfilt_bwd(dt, B, T, _p(tb), b.shape[-1], _p(ta), a.shape[-1], int(b.ndim == 1),
                                  capi.PADMODES[padmode], padlen, _p(tx), _p(tg), _p(gx), _p(gb), _p(ga), _p(sc),
                                  sc.numel(), _p(ws), need, _stream())
        assert rc == capi.PHS_OK, lib.phs_error_string(rc)
        torch.cuda.synchronize()
    finally:
        lib.phs_debug_set_spin_limit(0)
    if not coef:
        return gx.cpu().numpy()
    return gx.cpu().numpy(), gb.cpu().numpy(), ga.cpu().numpy()


def _oracle_jt(b, a, T, padmode, padlen):
    """The transposed Jacobian of the oracle's filtfilt for one filter (fp64):
    row k of filtfilt_ba(I) is the response to e_k, the column J[:, k]."""
    return oracle.filtfilt_ba(b, a, np.eye(T), padmode=padmode, padlen=padlen)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("padmode", MODES)
def test_filtfilt_bwd_capi_vs_oracle_jacobian(api, dtype, order, padmode):
    """grad_x = J^T grad_y with J the oracle's own filtfilt applied to unit
    impulses (exact for the linear map), shared and per-row filters, no pad,
    a one-sample pad, 9, and the largest allowed (T - 1)."""
    f64 = lambda v: np.asarray(v, np.float64)  # noqa: E731
    for B, T in ((3, 40), (2, 13), (1, 1)):
        for shared in (True, False):
            b, a, _ = _case(dtype, B, T, shared, D.seed_of("filtfilt-bwd-jt", dtype, order, padmode, T, shared),
                            order)
            gy = D.normal(D.rng(D.seed_of("filtfilt-bwd-jt-g", T)), (B, T), dtype)
            # 16 and 17: the pad kernels' LDS path and its global-memory one
            for padlen in sorted({0, min(1, T - 1), min(9, T - 1), min(16, T - 1), min(17, T - 1), T - 1}):
                gx = _run_bwd(api, b, a, gy, padmode, padlen)
                ref = np.stack([_oracle_jt(f64(b if shared else b[r]), f64(a if shared else a[r]), T, padmode,
                                           padlen) @ f64(gy[r]) for r in range(B)])
                D.check(gx, ref, f"B={B} T={T} shared={shared} padlen={padlen}", dtype=dtype)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("B,T", [(2, 3071), (3, 6145), (2, 12288), (1, 40000), (2, 30001)])
def test_filtfilt_bwd_capi_adjoint_identity(api, dtype, order, B, T):
    """<grad_y, F x> = <F^T grad_y, x> per row for two random x, F x the
    oracle's filtfilt in fp64, around and over tiles, every pad mode at
    padlen 9, T // 3 and T - 1."""
    f64 = lambda v: np.asarray(v, np.float64)  # noqa: E731
    b, a, _ = _case(dtype, B, T, False, D.seed_of("filtfilt-bwd-adj", dtype, order, T), order)
    g = D.rng(D.seed_of("filtfilt-bwd-adj-g", dtype, order, T))
    gy = D.normal(g, (B, T), dtype)
    xs = [g.standard_normal((B, T)) for _ in range(2)]
    for padmode in MODES:
        for padlen in (9, T // 3, T - 1):
            gx = f64(_run_bwd(api, b, a, gy, padmode, padlen))
            assert np.isfinite(gx).all()
            for x in xs:
                y = oracle.filtfilt_ba(f64(b), f64(a), x, padmode=padmode, padlen=padlen)
                lhs, rhs = np.sum(f64(gy) * y, axis=1), np.sum(gx * x, axis=1)
                scale = np.sum(np.abs(f64(gy) * y), axis=1) + np.sum(np.abs(gx * x), axis=1)
                tol = 1e-4 if dtype == np.float32 else 1e-11
                assert np.all(np.abs(lhs - rhs) <= tol * scale), (padmode, padlen, lhs, rhs)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("padmode", MODES)
def test_filtfilt_bwd_capi_coef_vs_oracle_fd(api, dtype, order, padmode):
    """dL/db . V and dL/da . V for L = <grad_y, filtfilt(b, a, x)> against
    the central difference of the oracle's filtfilt in fp64 (random
    directions V), shared and per-row filters, b one tap short, padlen 0, 1,
    9 and T - 1, a row shorter than a tile and one of two tiles; grad_x
    against the oracle's Jacobian as above."""
    f64 = lambda v: np.asarray(v, np.float64)  # noqa: E731
    tile = 6144 if dtype == np.float32 else 3072
    for B, T in ((3, 40), (2, tile + 9)):
        for shared, short in ((True, False), (False, False), (False, True)):
            g = D.rng(D.seed_of("filtfilt-bwd-coef", dtype, order, padmode, T, shared, short))
            # poles within radius 0.9: nearer the circle, central differences lose the digits to pin with
            b, a = D.ba_coefs(g, () if shared else (B,), order, dtype, rhi=0.9)
            x = D.normal(g, (B, T), dtype)
            if short:
                b = np.ascontiguousarray(b[..., :-1])
            gy = D.normal(g, (B, T), dtype)
            for padlen in sorted({0, 1, 9, 16, 17, T - 1}):
                gx, gb, ga = _run_bwd(api, b, a, gy, padmode, padlen, x=x)
                assert np.isfinite(gb).all() and np.isfinite(ga).all()

                def loss(bv, av):
                    return float(np.sum(f64(gy) * oracle.filtfilt_ba(bv, av, f64(x), padmode=padmode, padlen=padlen)))

                for which, grad in (("b", gb), ("a", ga)):
                    V = g.standard_normal(grad.shape)
                    if which == "b":
                        L = lambda t: loss(f64(b) + t * V, f64(a))  # noqa: E731
                    else:
                        L = lambda t: loss(f64(b), f64(a) + t * V)  # noqa: E731
                    eps = 1e-5  # fourth-order stencil: truncation ~eps^4, rounding ~1e-16 |L| / eps
                    fd = (8 * (L(eps) - L(-eps)) - (L(2 * eps) - L(-2 * eps))) / (12 * eps)
                    got = float(np.sum(f64(grad) * V))
                    # the scale of the directional sum (its terms cancel where the loss's do)
                    scale = max(1.0, abs(fd), float(np.sum(np.abs(f64(grad) * V))))
                    rtol = 2e-4 if dtype == np.float32 else 1e-7
                    assert abs(got - fd) <= rtol * scale, (which, B, T, shared, short, padlen, got, fd, scale)
                if T <= 64:
                    ref = np.stack([_oracle_jt(f64(b if shared else b[r]), f64(a if shared else a[r]), T, padmode,
                                               padlen) @ f64(gy[r]) for r in range(B)])
                    D.check(gx, ref, f"grad x B={B} T={T} padlen={padlen}", dtype=dtype)
                else:
                    D.check(gx, _run_bwd(api, b, a, gy, padmode, padlen), "grad x with and without coefficients",
                            dtype=dtype)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("order", ORDERS)
def test_filtfilt_bwd_capi_forced_fallback(api, dtype, order):
    """A one-poll budget: the tiles of both adjoint passes compute their
    entry states from the row's prefix (pass 2's adjoint) or suffix (pass 1's)
    themselves; equal to the look-back's result."""
    b, a, _ = _case(dtype, 3, 40000, False, D.seed_of("filtfilt-bwd-fallback", dtype, order), order)
    gy = D.normal(D.rng(D.seed_of("filtfilt-bwd-fallback-g", dtype)), (3, 40000), dtype)
    ref = _run_bwd(api, b, a, gy, "reflect", 9)
    got = _run_bwd(api, b, a, gy, "reflect", 9, spin_limit=1)
    D.check(got, ref, "fallback", dtype=dtype)
    x = D.normal(D.rng(D.seed_of("filtfilt-bwd-fallback-x", dtype)), (3, 40000), dtype)
    ref = _run_bwd(api, b, a, gy, "replicate", 9, x=x)
    got = _run_bwd(api, b, a, gy, "replicate", 9, spin_limit=1, x=x)
    for gg, rr, nm in zip(got, ref, ("x", "b", "a")):
        D.check(gg, rr, f"fallback with coefficients, grad {nm}", dtype=dtype)


@pytest.mark.parametrize("order", [2, 4])
def test_filtfilt_capi_constant_row_full_size(api, order):
    """At the C4 size a constant row comes out scaled by H(1)^2 for every
    edge-value pad: both passes start in, and stay in, their steady state."""
    B, T = 16, 480000
    g = D.rng(D.seed_of("filtfilt-dc", order))
    b, a = D.ba_coefs(g, (B,), order, np.float64, rhi=0.98)
    h1 = b.sum(-1) / (1 + a.sum(-1))
    x = np.full((B, T), 0.75)
    for mode in ("replicate", "reflect", "circular"):
        y = _run(api, b, a, x, mode, 9)
        D.check(y, np.broadcast_to((h1 * h1 * 0.75)[:, None], (B, T)), f"constant row {mode}", dtype=np.float64)


def test_filtfilt_capi_linearity_full_size(api):
    """filtfilt is linear in x for a fixed filter and pad mode (the edge
    states scale with the row): f(2u - 3v) = 2 f(u) - 3 f(v) at the C4 size."""
    B, T = 16, 480000
    g = D.rng(D.seed_of("filtfilt-linear"))
    b, a = D.ba_coefs(g, (B,), 3, np.float64, rhi=0.98)
    u, v = g.standard_normal((B, T)), g.standard_normal((B, T))
    for mode in MODES:
        lhs = _run(api, b, a, 2 * u - 3 * v, mode, 9)
        rhs = 2 * _run(api, b, a, u, mode, 9) - 3 * _run(api, b, a, v, mode, 9)
        D.check(lhs, rhs, f"linearity {mode}", dtype=np.float64)


# ---------------------------------------------------------------- torch API
def _biquad(g, lead, dtype):
    sos = D.sos_coefs(g, lead, 1, np.float64, rhi=0.98)[..., 0, :]
    return sos[..., 0:3].astype(dtype), sos[..., 4:6].astype(dtype)


def test_filtfilt_route_choice(hip):
    import torch

    from philtorch_amd.lti import filtering

    g = D.rng(D.seed_of("filtfilt-route"))
    b, a = (torch.tensor(v, device="cuda") for v in _biquad(g, (3,), np.float32))
    x = torch.randn(3, 100, device="cuda")
    ok = {"unroll_factor": 1}
    assert filtering._fused_filtfilt_applies(b, a, x, "replicate", "tdf2", ok)
    assert filtering._fused_filtfilt_applies(b, a, x, None, "df2", ok)
    assert filtering._fused_filtfilt_applies(b[0], a[0], x[0], "circular", "tdf2", ok)
    assert not filtering._fused_filtfilt_applies(b, a, x, "replicate", "tdf2", {})
    assert not filtering._fused_filtfilt_applies(b, a, x, "odd", "tdf2", ok)
    assert not filtering._fused_filtfilt_applies(b, a, x[:2], "replicate", "tdf2", ok)
    assert filtering._fused_filtfilt_applies(b[:, :2], a[:, :1], x, "replicate", "tdf2", ok)
    b4, a4 = (torch.tensor(v, device="cuda") for v in D.ba_coefs(g, (3,), 4, np.float32))
    assert filtering._fused_filtfilt_applies(b4, a4, x, "replicate", "tdf2", ok)
    assert filtering._fused_filtfilt_applies(torch.ones(3, 5, device="cuda"), a, x, "replicate", "tdf2", ok)
    assert not filtering._fused_filtfilt_applies(torch.ones(3, 6, device="cuda"), a, x, "replicate", "tdf2", ok)
    assert not filtering._fused_filtfilt_applies(b, torch.ones(3, 5, device="cuda"), x, "replicate", "tdf2", ok)
    # gradients w.r.t. x, b and a run philtorch::filtfilt_backward
    assert filtering._fused_filtfilt_applies(b, a, x.requires_grad_(), "replicate", "tdf2", ok)
    assert filtering._fused_filtfilt_applies(b.clone().requires_grad_(), a, x, "replicate", "tdf2", ok)
    assert filtering._fused_filtfilt_applies(b, a.clone().requires_grad_(), x, "replicate", "tdf2", ok)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_filtfilt_api_matches_scipy(hip, dtype):
    import scipy.signal as sg
    import torch

    from philtorch_amd.lti import filtering

    g = D.rng(D.seed_of("filtfilt-api", dtype))
    for shape, batched, order in (((3, 5000), False, 2), ((3, 5000), True, 2), ((777,), False, 2),
                                  ((3, 5000), True, 1), ((3, 5000), False, 1), ((3, 5000), True, 3),
                                  ((3, 5000), False, 4), ((3, 5000), True, 4)):
        b, a = D.ba_coefs(g, (shape[0],) if batched else (), order, np.float64, rhi=0.98)
        x = g.standard_normal(shape)
        tb, ta, tx = (torch.tensor(v.astype(dtype), device="cuda") for v in (b, a, x))
        for padmode, padlen, padtype in (("replicate", None, "constant"), ("reflect", 100, "even"),
                                         (None, None, None)):
            for form in ("tdf2", "df2"):
                assert filtering._fused_filtfilt_applies(tb, ta, tx, padmode, form, {"unroll_factor": 1})
                y = hip.lti.filtfilt(tb, ta, tx, padmode=padmode, padlen=padlen, form=form, unroll_factor=1)
                if batched:
                    ref = np.stack([sg.filtfilt(b[r], np.r_[1.0, a[r]], x[r], padtype=padtype,
                                                padlen=padlen if padtype else None)
                                    for r in range(shape[0])])
                else:
                    ref = sg.filtfilt(b, np.r_[1.0, a], x, axis=-1, padtype=padtype,
                                      padlen=padlen if padtype else None)
                D.check(y.cpu().numpy(), ref.astype(dtype), f"{shape} {batched} {padmode} {form}")


def test_filtfilt_api_c4_size_matches_composed_route(hip, monkeypatch):
    """The benchmark's filtfilt pattern at the C4 size (B=16, T=480000, fp32,
    one filtfilt per section, padmode replicate, padlen 9), output and the
    gradients w.r.t. x and every section's b and a: the fused route against
    the composed one (padding, lfilter_zi, two lfilter passes, flips, and
    their autograd) run in fp64 on the same fp32 values."""
    import torch

    from philtorch_amd.lti import filtering

    g = D.rng(D.seed_of("filtfilt-c4"))
    B, T, S = 16, 480000, 8
    sos = torch.tensor(D.sos_coefs(g, (B,), S, np.float32, rhi=0.98), device="cuda")
    x = torch.tensor(g.standard_normal((B, T)).astype(np.float32), device="cuda")
    gy = torch.tensor(g.standard_normal((B, T)).astype(np.float32), device="cuda")
    outs = []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(filtering, "_fused_filtfilt_applies", lambda *a, **k: False)
        dt = torch.float32 if fused else torch.float64
        xr = x.to(dt).requires_grad_(True)
        sr = sos.to(dt).requires_grad_(True)
        y = xr
        for s in range(S):
            y = hip.lti.filtfilt(sr[:, s, :3], sr[:, s, 4:], y, padmode="replicate", padlen=9, unroll_factor=1)
        gx, gs = torch.autograd.grad(y, (xr, sr), gy.to(dt))
        outs.append((y.detach().cpu().numpy(), gx.cpu().numpy(), gs.cpu().numpy()))
    D.check(outs[0][0], outs[1][0], "8 filtfilts", dtype=np.float32)
    D.check(outs[0][1], outs[1][1], "8 filtfilts, grad x", dtype=np.float32)
    for s in range(S):
        for cols, nm in ((slice(0, 3), "b"), (slice(4, 6), "a")):
            D.check(outs[0][2][:, s, cols], outs[1][2][:, s, cols], f"8 filtfilts, grad {nm} of section {s}",
                    dtype=np.float32)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_filtfilt_api_gradients_fused_vs_composed(hip, dtype, monkeypatch):
    """lti.filtfilt with gradients wanted for x, b and a (together and
    apart) takes the fused route both ways and matches the composed
    route's autograd (every pad mode, orders 1-4, shared and per-row
    filters, 1D and 2D x)."""
    import torch

    from philtorch_amd.lti import filtering

    taken = []
    orig = filtering._fused_filtfilt_applies
    g = D.rng(D.seed_of("filtfilt-xgrad", dtype))
    for shape, batched, order in (((3, 5000), True, 2), ((3, 5000), False, 1), ((777,), False, 2),
                                  ((3, 5000), True, 3), ((2, 6145), False, 4), ((3, 4001), True, 4)):
        b, a = D.ba_coefs(g, (shape[0],) if batched else (), order, dtype, rhi=0.98)
        x = g.standard_normal(shape).astype(dtype)
        gy = g.standard_normal(shape).astype(dtype)
        tgy = torch.tensor(gy, device="cuda")
        for (padmode, padlen), want in zip((("replicate", None), ("reflect", 100), ("constant", 7),
                                            ("circular", 31), (None, None)),
                                           ((1, 1, 1), (0, 0, 1), (1, 0, 0), (0, 1, 1), (1, 1, 1))):
            res = []
            for fused in (True, False):
                monkeypatch.setattr(filtering, "_fused_filtfilt_applies",
                                    (lambda *a_: taken.append(orig(*a_)) or taken[-1]) if fused
                                    else (lambda *a_, **k_: False))
                ts = [torch.tensor(v, device="cuda", requires_grad=bool(w)) for v, w in zip((b, a, x), want)]
                y = hip.lti.filtfilt(*ts, padmode=padmode, padlen=padlen, unroll_factor=1)
                if fused:
                    assert taken[-1] is True
                grads = torch.autograd.grad(y, [t for t in ts if t.requires_grad], tgy)
                res.append((y.detach().cpu().numpy(), [gg.cpu().numpy() for gg in grads]))
            nm = f"{shape} batched={batched} order={order} {padmode} {padlen} want={want}"
            D.check(res[0][0], res[1][0], nm, dtype=dtype)
            for gf, gc, wn in zip(res[0][1], res[1][1], [n for n, w in zip("bax", want) if w]):
                D.check(gf, gc, f"{nm} grad {wn}", dtype=dtype)


def test_filtfilt_api_gradcheck(hip):
    """gradcheck of lti.filtfilt w.r.t. b, a and x (the fused route's
    coefficient mode), and the output with and without gradients."""
    import torch

    g = D.rng(D.seed_of("filtfilt-grad"))
    b, a = (torch.tensor(v, device="cuda", requires_grad=True) for v in _biquad(g, (2,), np.float64))
    x = torch.tensor(g.standard_normal((2, 40)), device="cuda", requires_grad=True)
    f = lambda b_, a_, x_: hip.lti.filtfilt(b_, a_, x_, padlen=5, unroll_factor=1)  # noqa: E731
    assert torch.autograd.gradcheck(f, (b, a, x))
    with torch.no_grad():
        fused = f(b, a, x)
    D.check(fused.cpu().numpy(), f(b, a, x).detach().cpu().numpy(), "no-grad vs grad route")


def test_filtfilt_op_gradcheck(hip):
    """First and second order through the op (fp64): w.r.t. x alone
    (filtfilt_backward, whose own gradient is filtfilt) and w.r.t. b, a and
    x (the coefficient mode; second order through the composed route)."""
    import torch

    g = D.rng(D.seed_of("filtfilt-gradcheck"))
    for order, batched in ((1, False), (2, True), (3, False), (4, True)):
        b, a = (torch.tensor(v, device="cuda") for v in D.ba_coefs(g, (2,) if batched else (), order, np.float64,
                                                                     rhi=0.9))
        x = torch.tensor(g.standard_normal((2, 30)), device="cuda", requires_grad=True)
        bg, ag = b.clone().requires_grad_(True), a.clone().requires_grad_(True)
        for mode, padlen in ((1, 5), (2, 7), (3, 4), (0, 3), (1, 0), (2, 29)):
            f = lambda x_: torch.ops.philtorch.filtfilt(b, a, x_, mode, padlen)  # noqa: E731
            assert torch.autograd.gradcheck(f, (x,))
            assert torch.autograd.gradgradcheck(f, (x,))
            f3 = lambda b_, a_, x_: torch.ops.philtorch.filtfilt(b_, a_, x_, mode, padlen)  # noqa: E731
            assert torch.autograd.gradcheck(f3, (bg, ag, x))
            assert torch.autograd.gradcheck(f3, (bg, a, x.detach()))
            # the states-keeping forward (what lti.filtfilt takes with coefficient gradients)
            fs = lambda b_, a_, x_: torch.ops.philtorch.filtfilt_states(b_, a_, x_, mode, padlen)[0]  # noqa: E731
            assert torch.autograd.gradcheck(fs, (bg, ag, x))
            # its kept buffers give the coefficient backward's results bit for bit
            y0 = torch.ops.philtorch.filtfilt(b, a, x.detach(), mode, padlen)
            ys, mid, h1, h2 = torch.ops.philtorch.filtfilt_states(b, a, x.detach(), mode, padlen)
            torch.testing.assert_close(ys, y0, rtol=1e-12, atol=1e-12)
            gy = torch.randn_like(y0)
            r0 = torch.ops.philtorch.filtfilt_backward(b, a, x.detach(), gy, mode, padlen, True)
            r1 = torch.ops.philtorch.filtfilt_backward(b, a, x.detach(), gy, mode, padlen, True, mid, h1, h2)
            assert all(torch.equal(u, v) for u, v in zip(r0, r1))
        # second order runs the composed route, whose F.pad backward accumulates with atomics on the GPU
        # (run-to-run differences of ~1e-11 relative on gradients up to ~1e4)
        assert torch.autograd.gradgradcheck(f3, (bg, ag, x), nondet_tol=1e-7)


def test_filtfilt_api_errors(hip):
    import torch

    b, a = torch.tensor([0.5, 0.2, 0.1], device="cuda"), torch.tensor([-0.5, 0.2], device="cuda")
    with pytest.raises(AssertionError, match="must be greater than pad length"):
        hip.lti.filtfilt(b, a, torch.randn(2, 9, device="cuda"), unroll_factor=1)
    with pytest.raises(RuntimeError, match="must be greater than pad length"):
        torch.ops.philtorch.filtfilt(b, a, torch.randn(2, 9, device="cuda"), 1, 9)
    with pytest.raises(RuntimeError, match="order 4 at most"):
        torch.ops.philtorch.filtfilt(torch.ones(6, device="cuda"), a, torch.randn(2, 90, device="cuda"), 1, 9)
    with pytest.raises(RuntimeError, match="order 4 at most"):
        torch.ops.philtorch.filtfilt(b, torch.ones(5, device="cuda"), torch.randn(2, 90, device="cuda"), 1, 9)


def test_filtfilt_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("filtfilt-opcheck"))
    sos = torch.tensor(D.sos_coefs(g, (), 1, np.float32), device="cuda")
    x = torch.tensor(g.standard_normal((2, 700)).astype(np.float32), device="cuda")
    b, a = sos[0, :3].contiguous(), sos[0, 4:].contiguous()
    torch.library.opcheck(torch.ops.philtorch.filtfilt.default, (b, a, x, 1, 9),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(torch.ops.philtorch.filtfilt_states.default, (b, a, x, 1, 9),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(torch.ops.philtorch.filtfilt.default,
                          (b.expand(2, 3).contiguous(), a[:1].expand(2, 1).contiguous(), x, 2, 0),
                          test_utils=("test_schema", "test_faketensor"))
    b4, a4 = (torch.tensor(v, device="cuda") for v in D.ba_coefs(g, (2,), 4, np.float32))
    torch.library.opcheck(torch.ops.philtorch.filtfilt.default, (b4, a4, x, 3, 15),
                          test_utils=("test_schema", "test_faketensor"))
    for bb, aa, mode, padlen in ((b, a, 1, 9), (b4, a4, 2, 15), (b4, a4, 0, 0)):
        for need_coef in (False, True):
            torch.library.opcheck(torch.ops.philtorch.filtfilt_backward.default,
                                  (bb, aa, x, x.flip(-1).contiguous(), mode, padlen, need_coef),
                                  test_utils=("test_schema", "test_faketensor"))
        torch.library.opcheck(torch.ops.philtorch.filtfilt.default,
                              (bb.clone().requires_grad_(), aa, x.clone().requires_grad_(), mode, padlen),
                              test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
