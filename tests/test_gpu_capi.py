"""GPU parity through the C ABI itself (ctypes -> libphilscan -> HIP kernels).

Device memory comes from torch; every call passes raw device pointers, sizes
and the current stream exactly as a C/C++ caller of include/philscan.h would.
Also covers the self-compute fallback of the look-back (forced with a tiny
poll budget through phs_debug_set_spin_limit), workspace reuse across calls of
different shapes, and the error codes.
"""
import ctypes

import numpy as np
import pytest

from tests import _data as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def api(hip):
    import torch

    from tests import capi

    lib = capi.load()
    dev = torch.device("cuda", 0)
    # one workspace for every call of this module, zero-filled once
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
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


def _run(api, op, A, shared, zi, x, gy, M=None):
    """Forward + backward of one op through the C ABI; returns numpy results.
    M: the state order, for the order-M ops (recurN, lti_recurN)."""
    import torch

    lib, ws, capi = api
    dt = capi.DTYPES[np.dtype(x.dtype)]
    B, T = x.shape[:2]
    tA, tz, tx, tg = _dev(A), _dev(zi), _dev(x), _dev(gy)
    y = torch.empty_like(tx)
    order = () if M is None else (M,)

    def size(backward):
        if M is None:
            return lib.phs_workspace_size(capi.OPS[op], dt, B, T, int(shared), backward)
        return lib.phs_workspace_size_n(capi.OPS_N[op], dt, M, B, T, int(shared), backward)

    need = size(1)
    need_fwd = lambda: size(0)  # noqa: E731
    assert 0 < need <= ws.numel()
    # the call gets exactly the reported size: an under-reported size fails it
    rc = getattr(lib, f"phs_{op}_fwd")(dt, *order, B, T, _p(tA), int(shared), _p(tz), _p(tx), _p(y), _p(ws),
                                       need_fwd(), _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    gA, gz, gx = torch.empty_like(tA), torch.empty_like(tz), torch.empty_like(tx)
    rc = getattr(lib, f"phs_{op}_bwd")(dt, *order, B, T, _p(tA), int(shared), _p(tz), _p(y), _p(tg), _p(gx),
                                       _p(gA), _p(gz), _p(ws), need, _stream())
    assert rc == capi.PHS_OK, lib.phs_error_string(rc)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (y, gA, gz, gx)]


def _case(op, B, T, dtype, shared, seed):
    g = D.rng(seed)
    if op == "recur":
        A = D.coef(g, (T,) if shared else (B, T), dtype)
        zi, x, gy = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype), D.normal(g, (B, T), dtype)
    elif op == "lti_recur":
        A = D.coef(g, (1,) if shared else (B,), dtype)
        zi, x, gy = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype), D.normal(g, (B, T), dtype)
    elif op == "recur2":
        A = D.biquad_A(g, (T,) if shared else (B, T), dtype)
        zi, x, gy = D.normal(g, (B, 2), dtype), D.normal(g, (B, T, 2), dtype), D.normal(g, (B, T, 2), dtype)
    else:
        A = D.biquad_A(g, () if shared else (B,), dtype)
        zi, x, gy = D.normal(g, (B, 2), dtype), D.normal(g, (B, T, 2), dtype), D.normal(g, (B, T, 2), dtype)
    return A, zi, x, gy


def _oracle(op, A, zi, x, gy):
    import oracle

    if op == "recur":
        y = oracle.recur(A, zi, x)
        return [y, *oracle.recur_bwd(A, zi, y, gy)]
    if op == "lti_recur":
        y = oracle.lti_recur(A, zi, x)
        return [y, *oracle.lti_recur_bwd(A, zi, y, gy)]
    if op == "recur2":
        y = oracle.recurN(A, zi, x)
        return [y, *oracle.recurN_bwd(A, zi, y, gy)]
    y = oracle.lti_recurN(A, zi, x)
    return [y, *oracle.lti_recurN_bwd(A, zi, y, gy)]


def _check(got, ref):
    for name, a, b in zip(("y", "grad_A", "grad_zi", "grad_x"), got, ref):
        D.check(a.reshape(b.shape), b, name)


CASES = [
    ("recur", 3, 20000, np.float32, False),
    ("recur", 2, 9001, np.float64, True),
    ("recur", 2, 5000, np.complex64, False),
    ("lti_recur", 4, 30000, np.complex64, False),
    ("lti_recur", 3, 7000, np.float64, True),
    ("recur2", 2, 6000, np.float32, False),
    ("recur2", 2, 3000, np.float64, True),
    ("lti_recur2", 3, 9000, np.float32, False),
    ("lti_recur2", 2, 4000, np.complex128, True),
]


@pytest.mark.parametrize("op,B,T,dtype,shared", CASES)
def test_capi_parity(api, op, B, T, dtype, shared):
    A, zi, x, gy = _case(op, B, T, dtype, shared, D.seed_of("capi", op, B, T, np.dtype(dtype).str, shared))
    _check(_run(api, op, A, zi=zi, x=x, gy=gy, shared=shared), _oracle(op, A, zi, x, gy))


@pytest.mark.parametrize("op,B,T,dtype,shared", CASES[::2] + [("recur", 2, 1 << 20, np.float32, False)])
def test_capi_lookback_fallback(api, op, B, T, dtype, shared):
    """With a poll budget of 1, waiting tiles fold their row's prefix from the
    inputs themselves; results must not change."""
    lib = api[0]
    A, zi, x, gy = _case(op, B, T, dtype, shared, D.seed_of("fallback", op, B, T, np.dtype(dtype).str))
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, op, A, zi=zi, x=x, gy=gy, shared=shared)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(got, _oracle(op, A, zi, x, gy))


# Thousands of rows: a row's predecessor tile is claimed more than half a
# resident grid earlier, so the look-back wave of the complex and 2x2 scans
# polls for it while the tile is still loading (early look-back).
MANY_ROWS = [
    ("lti_recur", 2048, 6000, np.complex64, False),
    ("recur", 2048, 5000, np.complex128, False),
    ("recur2", 1536, 4000, np.float32, False),
    ("lti_recur2", 2048, 5000, np.float64, True),
]


@pytest.mark.parametrize("op,B,T,dtype,shared", MANY_ROWS)
def test_capi_many_rows_early_lookback(api, op, B, T, dtype, shared):
    A, zi, x, gy = _case(op, B, T, dtype, shared, D.seed_of("rows", op, B, T, np.dtype(dtype).str, shared))
    _check(_run(api, op, A, zi=zi, x=x, gy=gy, shared=shared), _oracle(op, A, zi, x, gy))


@pytest.mark.parametrize("op,B,T,dtype,shared", MANY_ROWS[::2])
def test_capi_many_rows_fallback(api, op, B, T, dtype, shared):
    """Early look-back with a poll budget of 1: tiles fall back to folding
    their row prefix from the inputs."""
    lib = api[0]
    A, zi, x, gy = _case(op, B, T, dtype, shared, D.seed_of("rows-fb", op, B, T, np.dtype(dtype).str))
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, op, A, zi=zi, x=x, gy=gy, shared=shared)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(got, _oracle(op, A, zi, x, gy))


# Order-M entry points (M = 3, 4).  600 rows put the look-back wave in its
# early-polling mode; the others run the chain mode.
CASES_N = [
    ("recurN", 3, 3, 5000, np.float32, False),
    ("recurN", 4, 2, 3000, np.complex128, True),
    ("lti_recurN", 3, 600, 2000, np.float64, False),
    ("lti_recurN", 4, 2, 4000, np.complex64, True),
    ("recurN", 4, 600, 700, np.float32, False),
]


def _case_n(op, M, B, T, dtype, shared, seed):
    g = D.rng(seed)
    shape = ((T,) if shared else (B, T)) if op == "recurN" else (() if shared else (B,))
    A = D.stable_matrix(g, shape, M, dtype)
    return A, D.normal(g, (B, M), dtype), D.normal(g, (B, T, M), dtype), D.normal(g, (B, T, M), dtype)


def _oracle_n(op, A, zi, x, gy):
    import oracle

    fwd, bwd = (oracle.recurN, oracle.recurN_bwd) if op == "recurN" else (oracle.lti_recurN, oracle.lti_recurN_bwd)
    y = fwd(A, zi, x)
    return [y, *bwd(A, zi, y, gy)]


@pytest.mark.parametrize("op,M,B,T,dtype,shared", CASES_N)
def test_capi_order_n_parity(api, op, M, B, T, dtype, shared):
    A, zi, x, gy = _case_n(op, M, B, T, dtype, shared, D.seed_of("capi-n", op, M, B, T, np.dtype(dtype).str))
    _check(_run(api, op, A, zi=zi, x=x, gy=gy, shared=shared, M=M), _oracle_n(op, A, zi, x, gy))


@pytest.mark.parametrize("op,M,B,T,dtype,shared", CASES_N[::2])
def test_capi_order_n_fallback(api, op, M, B, T, dtype, shared):
    """Order-M scans with a poll budget of 1 (look-back fallback)."""
    lib = api[0]
    A, zi, x, gy = _case_n(op, M, B, T, dtype, shared, D.seed_of("capi-n-fb", op, M, B, T, np.dtype(dtype).str))
    lib.phs_debug_set_spin_limit(1)
    try:
        got = _run(api, op, A, zi=zi, x=x, gy=gy, shared=shared, M=M)
    finally:
        lib.phs_debug_set_spin_limit(0)
    _check(got, _oracle_n(op, A, zi, x, gy))


def test_capi_workspace_reuse_many_calls(api):
    """One workspace, many calls of changing shapes: the per-call tags must
    keep every call independent of the status words left by earlier ones."""
    for i, (B, T) in enumerate([(4, 70000), (1, 3), (7, 8193), (4, 70000), (2, 200000), (3, 5)]):
        A, zi, x, gy = _case("recur", B, T, np.float32, False, 500 + i)
        _check(_run(api, "recur", A, zi=zi, x=x, gy=gy, shared=False), _oracle("recur", A, zi, x, gy))


def test_capi_errors(api):
    import torch

    lib, ws, capi = api
    x = torch.zeros(2, 100, device="cuda")
    z = torch.zeros(2, device="cuda")
    y = torch.empty_like(x)
    s = _stream()
    need = lib.phs_workspace_size(0, 0, 2, 100, 0, 0)
    assert need > 0
    assert lib.phs_recur_fwd(0, 2, 100, _p(x), 0, _p(z), _p(x), _p(y), _p(ws), need - 1, s) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_recur_fwd(0, 2, 100, _p(x), 0, _p(z), _p(x), _p(y), None, 0, s) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_recur_fwd(9, 2, 100, _p(x), 0, _p(z), _p(x), _p(y), _p(ws), ws.numel(), s) == capi.PHS_ERR_DTYPE
    assert lib.phs_recur_fwd(0, -1, 100, _p(x), 0, _p(z), _p(x), _p(y), _p(ws), ws.numel(), s) == capi.PHS_ERR_INVALID
    assert lib.phs_recur_fwd(0, 2, 100, None, 0, _p(z), _p(x), _p(y), _p(ws), ws.numel(), s) == capi.PHS_ERR_INVALID
    # empty problems are a no-op
    assert lib.phs_recur_fwd(0, 0, 100, None, 0, None, None, None, None, 0, s) == capi.PHS_OK
    assert lib.phs_recur_fwd(0, 2, 0, None, 0, None, None, None, None, 0, s) == capi.PHS_OK
    assert b"workspace" in lib.phs_error_string(capi.PHS_ERR_WORKSPACE)


# Look-back past the first window: with phs_debug_set_aggregates_only every
# tile after a row's first publishes only its aggregate, so tile q folds all
# q - 1 aggregates back to tile 0's state, window after window (64 entries
# each, after a first window of 8 for scalar scans).  Rows of 100-170 tiles
# per algebra and tile shape.
AGG_ONLY = [
    ("recur", 2, 100 * 8192 + 5, np.float32, False),         # scalar LPV: 8192-step tiles
    ("recur", 2, 150 * 1536 + 7, np.complex64, False),       # complex LPV: 1536
    ("lti_recur", 2, 120 * 3072 + 1, np.complex64, False),   # complex LTI: 3072
    ("lti_recur", 3, 170 * 4096, np.float64, True),          # fp64 scalar: 4096
    ("recur2", 2, 150 * 1536 + 3, np.float32, False),        # 2x2 LPV: 1536
    ("lti_recur2", 2, 140 * 3072 + 9, np.float32, True),     # 2x2 LTI: 3072
    ("lti_recur2", 2, 170 * 384 + 1, np.complex128, False),  # complex 2x2: 384
]


@pytest.mark.parametrize("op,B,T,dtype,shared", AGG_ONLY)
def test_capi_aggregates_only_multi_window(api, op, B, T, dtype, shared):
    lib = api[0]
    A, zi, x, gy = _case(op, B, T, dtype, shared, D.seed_of("agg-only", op, B, T, np.dtype(dtype).str))
    print(f"aggregates-only {op} B={B} T={T} {np.dtype(dtype).name}", flush=True)
    lib.phs_debug_set_aggregates_only(1)
    try:
        got = _run(api, op, A, zi=zi, x=x, gy=gy, shared=shared)
    finally:
        lib.phs_debug_set_aggregates_only(0)
    _check(got, _oracle(op, A, zi, x, gy))


@pytest.mark.parametrize("op,M,B,T,dtype", [("recurN", 3, 2, 100 * 1536 + 1, np.float32),
                                            ("lti_recurN", 4, 2, 130 * 768 + 3, np.complex64)])
def test_capi_order_n_aggregates_only(api, op, M, B, T, dtype):
    lib = api[0]
    A, zi, x, gy = _case_n(op, M, B, T, dtype, False, D.seed_of("agg-only-n", op, M, B, T))
    print(f"aggregates-only {op} M={M} B={B} T={T} {np.dtype(dtype).name}", flush=True)
    lib.phs_debug_set_aggregates_only(1)
    try:
        got = _run(api, op, A, zi=zi, x=x, gy=gy, shared=False, M=M)
    finally:
        lib.phs_debug_set_aggregates_only(0)
    _check(got, _oracle_n(op, A, zi, x, gy))


# Tracing launches (phs_debug_trace_next_launch): the traced scan gives the
# untraced results bit for bit and one record per tile whose phase stamps
# run in order.
@pytest.mark.parametrize(
    "op,dtype,B,T,shared",
    [
        ("recur", np.float32, 3, 50001, False),
        ("recur", np.float64, 2, 30000, True),
        ("lti_recur", np.complex64, 3, 20000, False),
        ("recur2", np.float32, 2, 9000, False),
        ("lti_recur2", np.float32, 3, 12000, False),
    ],
)
def test_capi_trace_records(api, op, dtype, B, T, shared):
    import torch

    lib, ws, capi = api
    A, zi, x, gy = _case(op, B, T, dtype, shared, D.seed_of("trace", op, np.dtype(dtype).str))
    ref = _run(api, op, A, shared, zi, x, gy)
    rec = torch.zeros(4096 * 8, dtype=torch.int64, device="cuda")
    dt = capi.DTYPES[np.dtype(x.dtype)]
    tA, tz, tx, tg = _dev(A), _dev(zi), _dev(x), _dev(gy)
    y = torch.empty_like(tx)
    gA, gz, gx = torch.empty_like(tA), torch.empty_like(tz), torch.empty_like(tx)
    fwd = lambda: getattr(lib, f"phs_{op}_fwd")(dt, B, T, _p(tA), int(shared), _p(tz), _p(tx), _p(y),  # noqa: E731
                                                _p(ws), ws.numel(), _stream())
    bwd = lambda: getattr(lib, f"phs_{op}_bwd")(dt, B, T, _p(tA), int(shared), _p(tz), _p(y), _p(tg),  # noqa: E731
                                                _p(gx), _p(gA), _p(gz), _p(ws), ws.numel(), _stream())
    for direction in ("fwd", "bwd"):
        rec.zero_()
        if direction == "bwd":
            assert fwd() == capi.PHS_OK
        lib.phs_debug_trace_next_launch(_p(rec), rec.numel() // 8)
        assert (fwd if direction == "fwd" else bwd)() == capi.PHS_OK
        torch.cuda.synchronize()
        r = rec.view(-1, 8).cpu().numpy()
        tiles = int((r[:, 0] != 0).sum())
        assert tiles >= 2 * B, (direction, tiles)
        r = r[:tiles]
        assert (r[:, 7] == np.arange(tiles)).all()
        start, claimed, loaded, aggs, entry, stored = (r[:, i] for i in range(6))
        assert (start <= claimed).all() and (claimed <= loaded).all() and (loaded <= aggs).all()
        assert (aggs <= entry).all() and (entry <= stored).all()
        assert ((stored - start) < 100_000_000).all()  # under a second of 100 MHz ticks
    lib.phs_debug_trace_next_launch(None, 0)
    got = [t.cpu().numpy() for t in (y, gA, gz, gx)]
    for name, g, e in zip(("y", "grad_A", "grad_zi", "grad_x"), got, ref):
        assert np.array_equal(g, e), name
