"""GPU parity of the fused second-order-section cascade.

The C ABI entry points phs_sosfilt_fwd / phs_sosfilt_bwd (ctypes, raw device
pointers, the caller's stream) against the oracle's cascade, which chains one
philtorch lfilter(form="tdf2") per section (oracle.sosfilt / sosfilt_bwd,
pinned to scipy.signal.sosfilt and to autograd of a serial loop in
tests/test_oracle.py), evaluated in fp64 on the GPU's exact inputs.  Covers rows that end inside a tile, on a tile, and
shorter than a lane's chunk; one to eight sections (more through the API, which chains launches); shared and per-row
coefficients; initial states and a zf gradient; the forced look-back
fallback in both directions; the torch API (philtorch_amd.lti.sosfilt) against
scipy and the per-section lfilter route, at the benchmark's full C4 size.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests import _data as D

pytestmark = pytest.mark.gpu

# tiles: float32 30720 steps forward, 6144 backward; float64 14336 / 1536
SHAPES = [(1, 1), (2, 17), (3, 1536), (2, 3071), (2, 6144), (3, 6145), (2, 12288), (2, 20000), (2, 30720), (1, 40000),
          (2, 61441)]
SECTIONS = [1, 3, 8]
FLOATS = [np.float32, np.float64]


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


def _case(dtype, B, T, S, shared, with_zi, with_gzf, seed):
    g = D.rng(seed)
    sos = D.sos_coefs(g, () if shared else (B,), S, dtype)
    x = D.normal(g, (B, T), dtype)
    zi = D.normal(g, (B, S, 2), dtype) if with_zi else None
    gy = D.normal(g, (B, T), dtype)
    gzf = D.normal(g, (B, S, 2), dtype) if with_gzf else None
    return sos, x, zi, gy, gzf


def _run(api, sos, x, zi, gy, gzf, grad=True):
    """Forward + backward through the C ABI; numpy (y, zf, gsos, gzi, gx)."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    B, T = x.shape
    S = sos.shape[-2]
    shared = int(sos.ndim == 2)
    ts, tx, tg = _dev(sos), _dev(x), _dev(gy)
    tz = _dev(zi) if zi is not None else None
    tgz = _dev(gzf) if gzf is not None else None
    need_f = lib.phs_sosfilt_workspace_size(dt, B, T, S, 0)
    need = lib.phs_sosfilt_workspace_size(dt, B, T, S, 1)
    assert 0 < need_f <= need <= ws.numel()
    ck = torch.empty(lib.phs_sosfilt_ckpt_size(dt, B, T, S), dtype=torch.uint8, device="cuda")
    y = torch.empty_like(tx)
    zf = torch.empty((B, S, 2), dtype=tx.dtype, device="cuda")
    rc = lib.phs_sosfilt_fwd(dt, B, T, S, _p(ts), shared, _p(tz), _p(tx), _p(y), _p(zf), _p(ck), _p(ws), need_f,
                             _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    gx, gzi = torch.empty_like(tx), torch.empty((B, S, 2), dtype=tx.dtype, device="cuda")
    gs = torch.empty_like(ts) if grad else None
    rc = lib.phs_sosfilt_bwd(dt, B, T, S, _p(ts), shared, _p(tx) if grad else None, _p(ck) if grad else None,
                             _p(tg), _p(tgz), _p(gx), _p(gs), _p(gzi), _p(ws), need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    out = [y, zf, gs, gzi, gx]
    return [None if t is None else t.cpu().numpy() for t in out]


def _exact(*arrays):
    """fp32 inputs widened to fp64: the oracle then evaluates the reference's
    algorithm on exactly the GPU's inputs without fp32 rounding.  A high-gain
    8-section cascade leaves ~1e-4 of rounding in the fp32 reference's own
    coefficient gradients, so two fp32 evaluations may differ by twice the bar
    while each is within it of this value."""
    return [None if a is None else np.asarray(a, dtype=np.float64) for a in arrays]


def _check_all(got, sos, x, zi, gy, gzf, dtype, name):
    y, zf, gs, gzi, gx = got
    sos, x, zi, gy, gzf = _exact(sos, x, zi, gy, gzf)
    ry, rzf = oracle.sosfilt(sos, x, zi)
    D.check(y, ry, f"{name} y", dtype=dtype)
    # final states and their gradients on the scale of the signal they end
    D.check(zf, rzf, f"{name} zf", dtype=dtype, scale=np.max(np.abs(ry)))
    rgs, rgzi, rgx = oracle.sosfilt_bwd(sos, x, zi, gy, gzf)
    D.check(gx, rgx, f"{name} grad_x", dtype=dtype)
    D.check(gzi, rgzi, f"{name} grad_zi", dtype=dtype, scale=np.max(np.abs(rgx)))
    if gs is not None:
        rgs[..., 3] = 0
        D.check(gs, rgs, f"{name} grad_sos", dtype=dtype)


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("B,T", SHAPES)
@pytest.mark.parametrize("S", SECTIONS)
def test_sosfilt_capi_parity(api, dtype, B, T, S):
    for shared, with_zi, with_gzf in ((False, True, True), (True, False, False)):
        case = _case(dtype, B, T, S, shared, with_zi, with_gzf, D.seed_of("sos", dtype, B, T, S, shared))
        _check_all(_run(api, *case), *case, dtype, f"S={S} B={B} T={T} shared={shared}")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_sosfilt_capi_long_rows(api, dtype):
    """Rows of 80+ tiles: look-backs that fold a first window of 8 tiles and
    further windows of 64 when the inclusive states are not yet published."""
    case = _case(dtype, 2, 1_000_003, 3, False, True, True, D.seed_of("sos-long", dtype))
    _check_all(_run(api, *case), *case, dtype, "long rows")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_sosfilt_capi_no_coef_grad(api, dtype):
    sos, x, zi, gy, gzf = _case(dtype, 3, 7000, 4, False, True, True, D.seed_of("sos-nograd", dtype))
    y, zf, gs, gzi, gx = _run(api, sos, x, zi, gy, gzf, grad=False)
    assert gs is None
    _, rgzi, rgx = oracle.sosfilt_bwd(*_exact(sos, x, zi, gy, gzf))
    D.check(gx, rgx, "grad_x", dtype=dtype)
    D.check(gzi, rgzi, "grad_zi", dtype=dtype, scale=np.max(np.abs(rgx)))


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_sosfilt_capi_forced_fallback(api, dtype):
    """A one-poll budget makes tiles compute their entry states from the row
    prefix (forward cascade) or suffix (adjoint cascade) themselves."""
    lib = api[0]
    # three forward tiles a row at float32's 30720-step tile
    case = _case(dtype, 2, 2 * 30720 + 5, 5, False, True, True, D.seed_of("sos-fallback", dtype))
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, *case)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check_all(got, *case, dtype, "fallback")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_sosfilt_capi_forced_kept_step(api, dtype):
    """Every kept_step branch of the eight-section gradient backward
    (phs_debug_set_sos_kept_step): none kept, so every re-derivation of a
    section's input runs from x through all sections below it; one and two
    kept slots at the steps the LDS allows (others return PHS_ERR_INVALID).
    grad_sos, grad_x and grad_zi against the oracle each time."""
    lib, _, capi = api
    case = _case(dtype, 3, 2 * 6144 + 77, 8, False, True, True, D.seed_of("sos-kept-step", dtype))
    ran = []
    try:
        for step in (0, 1, 2, 3, 4, 5, 7, 8):
            lib.phs_debug_set_sos_kept_step(step)
            print(f"sos kept_step={step} {np.dtype(dtype).name}", flush=True)
            try:
                got = _run(api, *case)
            except AssertionError as e:
                assert "invalid" in str(e).lower(), e  # the forced slots exceed this device's LDS
                assert step != 0
                continue
            _check_all(got, *case, dtype, f"kept_step={step}")
            ran.append(step)
    finally:
        lib.phs_debug_set_sos_kept_step(-1)
    assert 0 in ran and any(s not in (0, 8) for s in ran), ran


def test_sosfilt_capi_errors(api):
    import torch

    lib, ws, capi = api
    x = torch.zeros((2, 100), device="cuda")
    y = torch.empty_like(x)
    sos = torch.zeros((3, 6), device="cuda")
    args = (_p(sos), 1, None, _p(x), _p(y), None, None, _p(ws), ws.numel(), _stream())
    assert lib.phs_sosfilt_fwd(0, 2, 100, 0, *args) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_fwd(0, 2, 100, 9, *args) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_fwd(2, 2, 100, 3, *args) == capi.PHS_ERR_DTYPE
    need = lib.phs_sosfilt_workspace_size(0, 2, 100, 3, 0)
    assert lib.phs_sosfilt_fwd(0, 2, 100, 3, _p(sos), 1, None, _p(x), _p(y), None, None, _p(ws), need - 1,
                               _stream()) == capi.PHS_ERR_WORKSPACE
    # grad_sos without the forward's checkpoints
    assert lib.phs_sosfilt_bwd(0, 2, 100, 3, _p(sos), 1, _p(x), None, _p(x), None, _p(y), _p(sos), None, _p(ws),
                               ws.numel(), _stream()) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_workspace_size(0, 2, 100, 0, 0) == 0
    assert lib.phs_sosfilt_ckpt_size(2, 2, 100, 3) == 0


# ---------------------------------------------------------------- torch API
@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_sosfilt_api_matches_scipy(hip, dtype):
    import scipy.signal as sg
    import torch

    g = D.rng(D.seed_of("sos-api", dtype))
    for S, shape in ((4, (3, 5000)), (20, (2, 9000)), (2, (777,))):
        sos = D.sos_coefs(g, (), S, np.float64)
        sos[:, :3] *= 0.7
        sos[:, 3:] *= 1.3  # a0 != 1: normalised per section
        x = g.standard_normal(shape)
        zi = g.standard_normal((S,) + shape[:-1] + (2,))
        ry, rzf = sg.sosfilt(sos / sos[:, 3:4], x, axis=-1, zi=zi)
        y, zf = hip.lti.sosfilt(torch.tensor(sos, dtype=torch.float64 if dtype == np.float64 else torch.float32,
                                             device="cuda"),
                                torch.tensor(x.astype(dtype), device="cuda"),
                                zi=torch.tensor(zi.astype(dtype), device="cuda"))
        D.check(y.cpu().numpy(), ry.astype(dtype), f"y S={S}")
        D.check(zf.cpu().numpy(), rzf.astype(dtype), f"zf S={S}")


def test_sosfilt_api_grad_matches_oracle(hip):
    import torch

    g = D.rng(D.seed_of("sos-api-grad"))
    B, T, S = 3, 9000, 6
    sos = D.sos_coefs(g, (B,), S, np.float64)
    x = g.standard_normal((B, T))
    zi = g.standard_normal((S, B, 2))
    gy = g.standard_normal((B, T))
    gzf = g.standard_normal((S, B, 2))
    ts = torch.tensor(sos, device="cuda", requires_grad=True)
    tx = torch.tensor(x, device="cuda", requires_grad=True)
    tz = torch.tensor(zi, device="cuda", requires_grad=True)
    y, zf = hip.lti.sosfilt(ts, tx, zi=tz)
    ((y * torch.tensor(gy, device="cuda")).sum() + (zf * torch.tensor(gzf, device="cuda")).sum()).backward()
    zi_b = np.transpose(zi, (1, 0, 2))
    rgs, rgzi, rgx = oracle.sosfilt_bwd(sos, x, zi_b, gy, np.transpose(gzf, (1, 0, 2)))
    # the API normalises by a0: d/d a0 of (sos / a0) at a0 = 1 is -sum of the row's other grads
    rgs[..., 3] = -np.sum(rgs * sos, axis=-1) + rgs[..., 3] * sos[..., 3]
    D.check(ts.grad.cpu().numpy(), rgs, "grad_sos")
    D.check(tz.grad.cpu().numpy(), np.transpose(rgzi, (1, 0, 2)), "grad_zi")
    D.check(tx.grad.cpu().numpy(), rgx, "grad_x")


def test_sosfilt_gradcheck(hip):
    import torch

    g = D.rng(D.seed_of("sos-gradcheck"))
    sos = torch.tensor(D.sos_coefs(g, (2,), 3, np.float64), device="cuda", requires_grad=True)
    x = torch.tensor(g.standard_normal((2, 40)), device="cuda", requires_grad=True)
    zi = torch.tensor(g.standard_normal((3, 2, 2)), device="cuda", requires_grad=True)
    assert torch.autograd.gradcheck(lambda s, a, z: hip.lti.sosfilt(s, a, zi=z), (sos, x, zi))


def test_sosfilt_opcheck(hip):
    import torch

    g = D.rng(D.seed_of("sos-opcheck"))
    sos = torch.tensor(D.sos_coefs(g, (), 3, np.float32), device="cuda", requires_grad=True)
    x = torch.tensor(g.standard_normal((2, 700)).astype(np.float32), device="cuda", requires_grad=True)
    zi = torch.tensor(g.standard_normal((2, 3, 2)).astype(np.float32), device="cuda", requires_grad=True)
    torch.library.opcheck(torch.ops.philtorch.sosfilt.default, (sos, zi, x))
    torch.library.opcheck(torch.ops.philtorch.sosfilt.default, (sos, None, x))


def test_sosfilt_c4_size_matches_lfilter_chain(hip):
    """At the benchmark's C4 size (B=16, T=480000, 8 sections, fp32) the fused
    cascade agrees with one lfilter(tdf2) per section (each a biquad on the
    state-space kernel forward and the cascade kernel at one section
    backward), forward and backward: the two HIP routes against each other;
    tests/test_gpu_configs.py::test_c4_api_config checks the lfilter route
    against the oracle at this size."""
    import torch

    g = D.rng(D.seed_of("sos-c4"))
    B, T, S = 16, 480000, 8
    sos_np = D.sos_coefs(g, (B,), S, np.float32, rhi=0.98)
    x_np = g.standard_normal((B, T)).astype(np.float32)
    gy = torch.tensor(g.standard_normal((B, T)).astype(np.float32), device="cuda")
    res = []
    for fused in (True, False):
        sos = torch.tensor(sos_np, device="cuda", requires_grad=True)
        x = torch.tensor(x_np, device="cuda", requires_grad=True)
        if fused:
            y = hip.lti.sosfilt(sos, x)
        else:
            y = x
            for s in range(S):
                y = hip.lti.lfilter(sos[:, s, :3], sos[:, s, 4:], y, form="tdf2", unroll_factor=1)
        (y * gy).sum().backward()
        res.append((y.detach().cpu().numpy(), x.grad.cpu().numpy(), sos.grad.cpu().numpy()))
        del y, sos, x
    (y1, gx1, gs1), (y2, gx2, gs2) = res
    D.check(y1, y2, "y")
    D.check(gx1, gx2, "grad_x")
    gs2[..., 3] = gs1[..., 3]  # the lfilter chain does not differentiate a0
    D.check(gs1, gs2, "grad_sos")


# ---------------------------------------------------------------- lfilter route
def _biquad(g, lead, dtype):
    sos = D.sos_coefs(g, lead, 1, np.float64)[..., 0, :]
    return sos[..., 0:3].astype(dtype), sos[..., 4:6].astype(dtype)


def test_lfilter_tdf2_biquad_takes_fused_route(hip):
    import torch

    from philtorch_amd.lti import filtering

    g = D.rng(D.seed_of("lfilter-route"))
    b, a = (torch.tensor(v, device="cuda") for v in _biquad(g, (3,), np.float32))
    x = torch.randn(3, 100, device="cuda")
    assert filtering._fused_biquad_applies(b, a, x, None, "tdf2", {"unroll_factor": 1})
    assert not filtering._fused_biquad_applies(b, a, x, None, "df2", {"unroll_factor": 1})
    assert not filtering._fused_biquad_applies(b, a, x, None, "tdf2", {})
    assert not filtering._fused_biquad_applies(b, a, x.cpu(), None, "tdf2", {"unroll_factor": 1})


@pytest.mark.parametrize("batched", [False, True])
def test_lfilter_fused_route_matches_reference_route(hip, batched):
    """lfilter(tdf2, unroll_factor=1) on HIP (fused kernel) against the same
    call on CPU (the reference's pure-PyTorch route), with zi/zf, and filtfilt
    built on it."""
    import torch

    g = D.rng(D.seed_of("lfilter-fused", batched))
    b, a = _biquad(g, (4,) if batched else (), np.float64)
    x = g.standard_normal((4, 7000))
    zi = g.standard_normal((4, 2))
    tb, ta, tx, tz = (torch.tensor(v) for v in (b, a, x, zi))
    yg, zfg = hip.lti.lfilter(tb.cuda(), ta.cuda(), tx.cuda(), zi=tz.cuda(), unroll_factor=1)
    yc, zfc = hip.lti.lfilter(tb, ta, tx, zi=tz, unroll_factor=1)
    D.check(yg.cpu().numpy(), yc.numpy(), "y")
    D.check(zfg.cpu().numpy(), zfc.numpy(), "zf", scale=np.max(np.abs(yc.numpy())))
    fg = hip.lti.filtfilt(tb.cuda(), ta.cuda(), tx.cuda(), unroll_factor=1)
    fc = hip.lti.filtfilt(tb, ta, tx, unroll_factor=1)
    D.check(fg.cpu().numpy(), fc.numpy(), "filtfilt")


def test_lfilter_fused_route_second_order_gradients(hip):
    """Double backward through the fused route (its create_graph fallback is
    the differentiable per-section chain) and forward-mode AD (which keeps
    the reference's route)."""
    import torch
    import torch.autograd.forward_ad as fwad

    g = D.rng(D.seed_of("lfilter-fused-grad"))
    b, a = (torch.tensor(v, device="cuda", requires_grad=True) for v in _biquad(g, (2,), np.float64))
    x = torch.tensor(g.standard_normal((2, 30)), device="cuda", requires_grad=True)
    zi = torch.tensor(g.standard_normal((2, 2)), device="cuda", requires_grad=True)
    f = lambda b_, a_, x_, z_: hip.lti.lfilter(b_, a_, x_, zi=z_, unroll_factor=1)  # noqa: E731
    assert torch.autograd.gradcheck(f, (b, a, x, zi))
    assert torch.autograd.gradgradcheck(f, (b, a, x, zi))
    sos = torch.tensor(D.sos_coefs(g, (), 2, np.float64), device="cuda", requires_grad=True)
    assert torch.autograd.gradgradcheck(lambda s_, x_: hip.lti.sosfilt(s_, x_), (sos, x))
    with fwad.dual_level():
        xd = fwad.make_dual(x.detach(), torch.ones_like(x))
        y = hip.lti.lfilter(b.detach(), a.detach(), xd, unroll_factor=1)
        tangent = fwad.unpack_dual(y).tangent
    ref = hip.lti.lfilter(b.detach(), a.detach(), torch.ones_like(x), unroll_factor=1)
    D.check(tangent.cpu().numpy(), ref.cpu().numpy(), "jvp")


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_sosfilt_capi_aggregates_only_multi_window(api, dtype):
    """Tiles after a row's first publish aggregates only (testing hook): every
    section's look-back folds back to tile 0 through windows of 64 entries
    (70+ tiles per row at the forward's tile, more at the backward's),
    forward cascade and adjoint cascade."""
    lib = api[0]
    T = 70 * (30720 if dtype == np.float32 else 14336) + 3
    case = _case(dtype, 2, T, 3, False, True, True, D.seed_of("sos-agg-only", dtype))
    lib.phs_debug_set_aggregates_only(1)
    try:
        got = _run(api, *case)
    finally:
        lib.phs_debug_set_aggregates_only(0)
    _check_all(got, *case, dtype, "aggregates only")


# ---------------------------------------------------------------- one biquad from b and a
@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("layout", ["table", "rows", "shared"])
@pytest.mark.parametrize("nb", [1, 2, 3])
def test_biquad_capi_reads_b_and_a_in_place(api, dtype, layout, nb):
    """phs_biquad_fwd/bwd: b and a read where they lie (columns of a
    [B, S, 3] / [B, S, 2] coefficient table at row stride S*3 / S*2,
    contiguous rows, or one shared filter) against the oracle's cascade at
    S = 1, with initial and final states and the coefficient gradients."""
    import torch

    lib, ws, capi = api
    g = D.rng(D.seed_of("biquad-capi", np.dtype(dtype).str, layout, nb))
    B, T = 3, 13001
    dt = capi.DTYPES[np.dtype(dtype)]
    sos = D.sos_coefs(g, (B, 4), 1, dtype)[..., 0, :] if layout == "table" else \
        D.sos_coefs(g, () if layout == "shared" else (B,), 1, dtype)[..., 0, :]
    if nb < 3:
        sos[..., nb:3] = 0
    x, gy = D.normal(g, (B, T), dtype), D.normal(g, (B, T), dtype)
    zi, gzf = D.normal(g, (B, 2), dtype), D.normal(g, (B, 2), dtype)
    tsos = _dev(sos)
    if layout == "table":  # column s = 2 of the table: row stride 4 * 6 elements
        tb, ta = tsos[:, 2, 0:nb], tsos[:, 2, 4:6]
        sos_rows = sos[:, 2]
    else:
        tb, ta = tsos[..., 0:nb], tsos[..., 4:6]
        sos_rows = sos
    bs = 0 if tb.dim() == 1 else tb.stride(0)
    as_ = 0 if ta.dim() == 1 else ta.stride(0)
    tx, tg, tz, tgz = _dev(x), _dev(gy), _dev(zi), _dev(gzf)
    need = lib.phs_sosfilt_workspace_size(dt, B, T, 1, 1)
    ck = torch.empty(lib.phs_sosfilt_ckpt_size(dt, B, T, 1), dtype=torch.uint8, device="cuda")
    y, zf = torch.empty_like(tx), torch.empty((B, 2), dtype=tx.dtype, device="cuda")
    print(f"biquad capi {np.dtype(dtype).name} layout={layout} nb={nb}", flush=True)
    rc = lib.phs_biquad_fwd(dt, B, T, _p(tb), nb, bs, _p(ta), as_, _p(tz), _p(tx), _p(y), _p(zf), _p(ck), _p(ws),
                            need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    rows = 1 if layout == "shared" else B
    gx, gzi = torch.empty_like(tx), torch.empty((B, 2), dtype=tx.dtype, device="cuda")
    gb = torch.full((rows, nb), float("nan"), dtype=tx.dtype, device="cuda")
    ga = torch.full((rows, 2), float("nan"), dtype=tx.dtype, device="cuda")
    rc = lib.phs_biquad_bwd(dt, B, T, _p(tb), nb, bs, _p(ta), as_, _p(tx), _p(ck), _p(tg), _p(tgz), _p(gx), _p(gb),
                            _p(ga), _p(gzi), _p(ws), need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    full = np.asarray(sos_rows, np.float64)[..., None, :]  # (B|., 1, 6)
    got = [y.cpu().numpy(), zf.cpu().numpy()[:, None, :], None, gzi.cpu().numpy()[:, None, :], gx.cpu().numpy()]
    _check_all(got, full, x, zi[:, None, :], gy, gzf[:, None, :], dtype, f"biquad {layout}")
    rgs, _, _ = oracle.sosfilt_bwd(*_exact(full, x, zi[:, None, :], gy, gzf[:, None, :]))
    rgs = rgs.reshape(rows, 6)
    D.check(gb.cpu().numpy(), rgs[:, 0:nb], "grad_b", dtype=dtype)
    D.check(ga.cpu().numpy(), rgs[:, 4:6], "grad_a", dtype=dtype)
    # phs_biquad_bwd_cols: the same gradients written as whole tables, the
    # biquad's column in place (bit-identical: the same reduction) and zeros
    # in every other column
    gbt = torch.full((rows, 5, nb), float("nan"), dtype=tx.dtype, device="cuda")
    gat = torch.full((rows, 2, 2), float("nan"), dtype=tx.dtype, device="cuda")
    gx2, gzi2 = torch.empty_like(tx), torch.empty((B, 2), dtype=tx.dtype, device="cuda")
    print(f"biquad capi cols {np.dtype(dtype).name} layout={layout} nb={nb}", flush=True)
    rc = lib.phs_biquad_bwd_cols(dt, B, T, _p(tb), nb, bs, _p(ta), as_, _p(tx), _p(ck), _p(tg), _p(tgz), _p(gx2),
                                 _p(gbt), 5, 3, _p(gat), 2, 1, _p(gzi2), _p(ws), need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(gbt[:, 3], gb) and torch.equal(gat[:, 1], ga)
    assert torch.equal(gx2, gx) and torch.equal(gzi2, gzi)
    others = torch.cat([gbt[:, [0, 1, 2, 4]].flatten(), gat[:, 0].flatten()])
    assert torch.equal(others, torch.zeros_like(others))
    for bc, bcol, ac, acol in ((5, 5, 2, 1), (5, -1, 2, 1), (0, 0, 2, 1), (5, 3, 2, 2)):
        rc = lib.phs_biquad_bwd_cols(dt, B, T, _p(tb), nb, bs, _p(ta), as_, _p(tx), _p(ck), _p(tg), _p(tgz),
                                     _p(gx2), _p(gbt), bc, bcol, _p(gat), ac, acol, _p(gzi2), _p(ws), need,
                                     _stream())
        assert rc == capi.PHS_ERR_INVALID


@pytest.mark.parametrize("dtype", FLOATS, ids=lambda d: np.dtype(d).name)
def test_biquad_forward_checkpoints_match_cascade_kernel(api, dtype):
    """phs_biquad_fwd runs the state-space kernel's pass and writes the
    checkpoints the cascade backward reads: the state entering every 32nd
    step (float32; float64 every 8th), the same values phs_sosfilt_fwd's
    cascade kernel at S = 1 writes for the same filter (to the parity bar),
    with equal outputs and zf.  Every checkpoint is written (none stays NaN)."""
    import torch

    lib, ws, capi = api
    g = D.rng(D.seed_of("biquad-ckpt", np.dtype(dtype).str))
    B, T = 3, 3 * 6144 + 77
    dt = capi.DTYPES[np.dtype(dtype)]
    sos = D.sos_coefs(g, (B,), 1, dtype)  # (B, 1, 6)
    x, zi = D.normal(g, (B, T), dtype), D.normal(g, (B, 1, 2), dtype)
    tsos, tx, tz = _dev(sos), _dev(x), _dev(zi)
    need = lib.phs_sosfilt_workspace_size(dt, B, T, 1, 0)
    nck = lib.phs_sosfilt_ckpt_size(dt, B, T, 1)
    outs = []
    for route in ("biquad", "sosfilt"):
        ck = torch.full((nck // 8,), float("nan"), dtype=torch.float64, device="cuda")
        y, zf = torch.empty_like(tx), torch.empty((B, 1, 2), dtype=tx.dtype, device="cuda")
        print(f"biquad ckpt {np.dtype(dtype).name} {route}", flush=True)
        if route == "biquad":
            tb, ta = tsos[:, 0, 0:3], tsos[:, 0, 4:6]
            rc = lib.phs_biquad_fwd(dt, B, T, _p(tb), 3, tb.stride(0), _p(ta), ta.stride(0), _p(tz), _p(tx), _p(y),
                                    _p(zf), _p(ck), _p(ws), need, _stream())
        else:
            rc = lib.phs_sosfilt_fwd(dt, B, T, 1, _p(tsos), 0, _p(tz), _p(tx), _p(y), _p(zf), _p(ck), _p(ws), need,
                                     _stream())
        assert rc == capi.PHS_OK, lib.phs_error_string(rc)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (ck, y, zf)])
    (ck1, y1, zf1), (ck2, y2, zf2) = outs
    assert np.isfinite(ck1).all() and np.isfinite(ck2).all()
    every = 32 if dtype == np.float32 else 8
    assert ck1.size == B * ((T + every - 1) // every) * 2
    D.check(ck1, ck2, "ckpt", dtype=dtype)
    D.check(y1, y2, "y", dtype=dtype)
    D.check(zf1, zf2, "zf", dtype=dtype)


def test_lfilter_columns_hand_gradients_to_tables(hip):
    """The C4 caller pattern's b[:, s] / a[:, s] of coefficient tables
    take philtorch::biquad_cols, whose backward writes the tables' gradients
    whole: the gradients w.r.t. x and the tables are bit-identical to the
    plain route's (the same columns passed as fresh tensors), also for 1-D
    shared tables and for a table of b beside a plain a; views that retain
    their gradient keep the plain route."""
    import torch

    from philtorch_amd import lti
    from philtorch_amd.lti import filtering

    g = D.rng(D.seed_of("biquad-cols-route"))
    B, T, S = 3, 7001, 4
    for shared in (False, True):
        lead = (S,) if shared else (B, S)
        sos = D.sos_coefs(g, lead, 1, np.float64)[..., 0, :]
        x0 = torch.tensor(g.standard_normal((B, T)), device="cuda")
        gy = torch.tensor(g.standard_normal((B, T)), device="cuda")
        grads = {}
        for route in ("cols", "plain", "mixed"):
            print(f"biquad cols route={route} shared={shared}", flush=True)
            bt = torch.tensor(sos[..., 0:3], device="cuda").requires_grad_(True)
            at = torch.tensor(sos[..., 4:6], device="cuda").requires_grad_(True)
            x = x0.clone().requires_grad_(True)
            y = x
            for s in range(S):
                bs, as_ = bt[..., s, :], at[..., s, :]
                if route == "cols":
                    assert filtering._table_column(bs)[1] == s and filtering._table_column(as_)[1] == s
                if route in ("plain", "mixed"):
                    as_ = as_ * 1.0  # not a view: the plain route for a
                if route == "plain":
                    bs = bs * 1.0
                y = lti.lfilter(bs, as_, y, form="tdf2", unroll_factor=1)
            grads[route] = torch.autograd.grad(y, (x, bt, at), gy)
        for route in ("plain", "mixed"):
            for got, ref in zip(grads[route], grads["cols"]):
                assert torch.equal(got, ref), route
        # against the oracle's cascade (every section a column of the tables)
        full = np.broadcast_to(sos, (B, S, 6)) if shared else sos
        rgs, _, rgx = oracle.sosfilt_bwd(*_exact(full, x0.cpu().numpy(), None, gy.cpu().numpy(), None))
        gsum = rgs.sum(0) if shared else rgs
        D.check(grads["cols"][0].cpu().numpy(), rgx, "grad_x", dtype=np.float64)
        D.check(grads["cols"][1].cpu().numpy(), gsum[..., 0:3], "grad_b table", dtype=np.float64)
        D.check(grads["cols"][2].cpu().numpy(), gsum[..., 4:6], "grad_a table", dtype=np.float64)
    bt = torch.zeros((B, S, 3), device="cuda", requires_grad=True)
    v = bt[:, 1]
    v.retain_grad()
    assert filtering._table_column(v)[1] == -1


def test_biquad_cols_op_gradients_and_opcheck(hip):
    """philtorch::biquad_cols: gradcheck of the fused table gradients,
    gradgradcheck of the composite, opcheck."""
    import torch

    g = D.rng(D.seed_of("biquad-cols-op"))
    B, T = 2, 40
    tab_b = torch.tensor(g.standard_normal((B, 4, 3)), device="cuda", requires_grad=True)
    tab_a = torch.tensor(D.sos_coefs(g, (B, 4), 1, np.float64)[..., 0, 4:6], device="cuda").requires_grad_(True)
    a_row = torch.tensor(D.sos_coefs(g, (B,), 1, np.float64)[..., 0, 4:6], device="cuda").requires_grad_(True)
    x = torch.tensor(g.standard_normal((B, T)), device="cuda", requires_grad=True)
    zi = torch.tensor(g.standard_normal((B, 2)), device="cuda", requires_grad=True)
    f = lambda tb_, ta_, z_, x_: torch.ops.philtorch.biquad_cols(tb_, 2, ta_, 1, z_, x_)[:2]  # noqa: E731
    assert torch.autograd.gradcheck(f, (tab_b, tab_a, zi, x))
    assert torch.autograd.gradgradcheck(f, (tab_b, tab_a, zi, x))
    f2 = lambda tb_, a_, x_: torch.ops.philtorch.biquad_cols(tb_, 0, a_, -1, None, x_)[0]  # noqa: E731
    assert torch.autograd.gradcheck(f2, (tab_b, a_row, x))
    # the same through lti.lfilter, whose column route is its own autograd
    # Function over the same ops (first and second order)
    from philtorch_amd import lti

    f3 = lambda tb_, ta_, z_, x_: lti.lfilter(tb_[:, 2], ta_[:, 1], x_, zi=z_, form="tdf2", unroll_factor=1)  # noqa: E731
    assert torch.autograd.gradcheck(f3, (tab_b, tab_a, zi, x))
    assert torch.autograd.gradgradcheck(f3, (tab_b, tab_a, zi, x))
    s = lambda v: torch.tensor(np.asarray(v, np.float32), device="cuda")  # noqa: E731
    torch.library.opcheck(torch.ops.philtorch.biquad_cols.default,
                          (s(g.standard_normal((3, 3))), 1, s([[-0.5, 0.2]] * 3), 2, None,
                           s(g.standard_normal((B, 700)))),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))


def test_biquad_op_gradients_and_opcheck(hip):
    """philtorch::biquad through autograd: strided columns of a coefficient
    table (the C4 caller pattern), gradcheck (the fused backward),
    gradgradcheck (the composite), opcheck."""
    import torch

    g = D.rng(D.seed_of("biquad-op"))
    B, T = 2, 40
    sos = torch.tensor(D.sos_coefs(g, (B, 3), 1, np.float64)[..., 0, :], device="cuda")
    b = sos[:, 1, 0:3].clone().requires_grad_(True)
    a = sos[:, 1, 4:6].clone().requires_grad_(True)
    x = torch.tensor(g.standard_normal((B, T)), device="cuda", requires_grad=True)
    zi = torch.tensor(g.standard_normal((B, 2)), device="cuda", requires_grad=True)
    f = lambda b_, a_, z_, x_: torch.ops.philtorch.biquad(b_, a_, z_, x_)[:2]  # noqa: E731
    assert torch.autograd.gradcheck(f, (b, a, zi, x))
    assert torch.autograd.gradgradcheck(f, (b, a, zi, x))
    tab_b = torch.tensor(g.standard_normal((B, 4, 3)), device="cuda", requires_grad=True)
    tab_a = (torch.tensor(D.sos_coefs(g, (B, 4), 1, np.float64)[..., 0, 4:6], device="cuda")).requires_grad_(True)
    f2 = lambda tb_, ta_, x_: torch.ops.philtorch.biquad(tb_[:, 2], ta_[:, 2], None, x_)[0]  # noqa: E731
    assert torch.autograd.gradcheck(f2, (tab_b, tab_a, x))
    s = lambda v: torch.tensor(np.asarray(v, np.float32), device="cuda")  # noqa: E731
    torch.library.opcheck(torch.ops.philtorch.biquad.default,
                          (s(g.standard_normal(3)), s([-0.5, 0.2]), None, s(g.standard_normal((B, 700)))),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
