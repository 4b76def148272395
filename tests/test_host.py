"""Host-side checks that need no GPU: the C ABI library, the op registrations
and fake kernels, and the pure-PyTorch routes of the Python API."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests import _data as D
from tests import capi


# ------------------------------------------------------------ C ABI library
def test_capi_exports_every_declared_symbol():
    lib = ctypes.CDLL(capi.LIB_PATH)
    declared = capi.declared_symbols()
    assert len(declared) >= 12
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, f"declared in include/philscan.h but not exported: {missing}"


def test_capi_host_only_calls():
    lib = capi.load()
    assert lib.phs_abi_version() == 112
    for op in capi.OPS.values():
        for dt in capi.DTYPES.values():
            fwd = lib.phs_workspace_size(op, dt, 64, 65536, 0, 0)
            bwd = lib.phs_workspace_size(op, dt, 64, 65536, 0, 1)
            assert 0 < fwd <= bwd
    assert lib.phs_workspace_size(0, 0, 0, 10, 0, 0) == 0
    assert lib.phs_workspace_size(7, 0, 4, 10, 0, 0) == 0
    assert lib.phs_workspace_size(0, 9, 4, 10, 0, 0) == 0
    # shared LPV backward needs per-step scratch for the batch reduction
    assert lib.phs_workspace_size(0, 0, 8, 1 << 20, 1, 1) > lib.phs_workspace_size(0, 0, 8, 1 << 20, 0, 1) + 8 * 4 * (1 << 20) - 4096
    for code in range(5):
        assert lib.phs_error_string(code)
    # argument errors are reported before anything is launched
    dummy = ctypes.c_void_p(16)
    assert lib.phs_recur_fwd(9, 2, 100, dummy, 0, dummy, dummy, dummy, dummy, 1 << 20, None) == capi.PHS_ERR_DTYPE
    assert lib.phs_recur_fwd(0, -1, 100, dummy, 0, dummy, dummy, dummy, dummy, 1 << 20, None) == capi.PHS_ERR_INVALID
    assert lib.phs_recur_fwd(0, 2, 100, None, 0, dummy, dummy, dummy, dummy, 1 << 20, None) == capi.PHS_ERR_INVALID
    assert lib.phs_recur_fwd(0, 2, 100, dummy, 0, dummy, dummy, dummy, None, 0, None) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_recur_bwd(0, 2, 100, dummy, 0, dummy, None, dummy, dummy, dummy, dummy, dummy, 1 << 20,
                             None) == capi.PHS_ERR_INVALID
    assert lib.phs_recur_fwd(0, 0, 100, None, 0, None, None, None, None, 0, None) == capi.PHS_OK


def test_capi_workspace_size_is_exact():
    """Each entry point accepts exactly the size phs_workspace_size(_n)
    reports and refuses one byte less.  Runs without a GPU only: with one,
    the accepted call would launch on dummy pointers."""
    if torch.cuda.device_count() > 0:
        pytest.skip("calls entry points with dummy pointers; CPU-only check")
    lib = capi.load()
    d = ctypes.c_void_p(16)
    fixed = [(name, code, None) for name, code in capi.OPS.items()]
    orders = [(name, code, M) for name, code in capi.OPS_N.items() for M in (1, 2, 3, 4)]
    for name, code, M in fixed + orders:
        for dt in capi.DTYPES.values():
            for shared in (0, 1):
                for B, T in ((3, 11), (5, 40000)):
                    order = () if M is None else (M,)
                    for bw in (0, 1):
                        if M is None:
                            n = lib.phs_workspace_size(code, dt, B, T, shared, bw)
                        else:
                            n = lib.phs_workspace_size_n(code, dt, M, B, T, shared, bw)
                        if bw:
                            call = lambda size: getattr(lib, f"phs_{name}_bwd")(  # noqa: E731
                                dt, *order, B, T, d, shared, d, d, d, d, d, d, d, size, None)
                        else:
                            call = lambda size: getattr(lib, f"phs_{name}_fwd")(  # noqa: E731
                                dt, *order, B, T, d, shared, d, d, d, d, size, None)
                        assert call(n - 1) == capi.PHS_ERR_WORKSPACE, (name, M, dt, shared, B, T, bw)
                        assert call(n) == capi.PHS_ERR_LAUNCH, (name, M, dt, shared, B, T, bw)  # no device here


def test_capi_order_n_host_only_calls():
    lib = capi.load()
    RECURN, LTI_RECURN = capi.OPS_N["recurN"], capi.OPS_N["lti_recurN"]
    for dt in capi.DTYPES.values():
        for bw in (0, 1):
            # orders 1 and 2 size exactly as the fixed-order ops
            assert lib.phs_workspace_size_n(RECURN, dt, 1, 8, 5000, 0, bw) == lib.phs_workspace_size(0, dt, 8, 5000, 0, bw)
            assert lib.phs_workspace_size_n(LTI_RECURN, dt, 2, 8, 5000, 1, bw) == lib.phs_workspace_size(3, dt, 8, 5000, 1, bw)
            for M in (3, 4):
                for op in (RECURN, LTI_RECURN):
                    assert lib.phs_workspace_size_n(op, dt, M, 8, 5000, 0, bw) > 0
        assert lib.phs_workspace_size_n(RECURN, dt, 5, 8, 5000, 0, 0) == 0
        assert lib.phs_workspace_size_n(RECURN, dt, 0, 8, 5000, 0, 0) == 0
    assert lib.phs_workspace_size_n(0, 0, 2, 8, 5000, 0, 0) == 0  # fixed-order op, wrong order
    assert lib.phs_workspace_size_n(2, 0, 2, 8, 5000, 0, 0) == lib.phs_workspace_size(2, 0, 8, 5000, 0, 0)
    assert lib.phs_workspace_size_n(RECURN, 0, 3, 0, 5000, 0, 0) == 0
    dummy = ctypes.c_void_p(16)
    for M in (0, 5):
        assert lib.phs_recurN_fwd(0, M, 2, 100, dummy, 0, dummy, dummy, dummy, dummy, 1 << 20, None) == capi.PHS_ERR_INVALID
        assert lib.phs_lti_recurN_bwd(0, M, 2, 100, dummy, 0, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                                      1 << 20, None) == capi.PHS_ERR_INVALID
    assert lib.phs_recurN_fwd(9, 3, 2, 100, dummy, 0, dummy, dummy, dummy, dummy, 1 << 20, None) == capi.PHS_ERR_DTYPE
    assert lib.phs_lti_recurN_fwd(0, 4, 2, 100, dummy, 0, dummy, dummy, dummy, None, 0, None) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_recurN_fwd(0, 3, 0, 100, None, 0, None, None, None, None, 0, None) == capi.PHS_OK


# ------------------------------------------------------------ op registration
def test_ops_registered_with_reference_schemas():
    import philtorch_amd  # noqa: F401

    for name in ("recur2", "recurN", "lti_recur2", "lti_recurN", "lti_recur", "recur"):
        schema = getattr(torch.ops.philtorch, name).default._schema
        assert str(schema) == f"philtorch::{name}(Tensor A, Tensor zi, Tensor x) -> Tensor"
        assert torch.Tag.pt2_compliant_tag in getattr(torch.ops.philtorch, name).default.tags
    for name in ("recur_backward", "recurN_backward", "lti_recur_backward", "lti_recurN_backward"):
        schema = str(getattr(torch.ops.philtorch, name).default._schema)
        assert schema.endswith("-> (Tensor, Tensor, Tensor)")


def test_cpu_key_serves_the_scan_ops_only():
    """The reference's ops, recur and the backward ops have CPU kernels (as
    the reference registers its CPU extension); the fused filter ops are
    HIP-only and raise on CPU tensors."""
    import philtorch_amd  # noqa: F401

    y = torch.ops.philtorch.recur(torch.zeros(2, 3), torch.ones(2), torch.ones(2, 3))
    assert y.tolist() == [[1.0, 1.0, 1.0]] * 2
    with pytest.raises(NotImplementedError):
        torch.ops.philtorch.sosfilt(torch.zeros(1, 6), None, torch.zeros(2, 3))


@pytest.mark.parametrize(
    "op,A,zi,x",
    [
        ("recur", (4, 100), (4,), (4, 100)),
        ("recur", (100,), (4,), (4, 100)),
        ("recurN", (4, 100, 2, 2), (4, 2), (4, 100, 2)),
        ("recur2", (100, 2, 2), (4, 2), (4, 100, 2)),
        ("lti_recur", (4,), (4,), (4, 100)),
        ("lti_recur", (), (4,), (4, 100)),
        ("lti_recur2", (4, 2, 2), (4, 2), (4, 100, 2)),
        ("lti_recurN", (3, 3), (4, 3), (4, 100, 3)),
    ],
)
def test_fake_kernels_shapes(op, A, zi, x):
    import philtorch_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        fa, fz, fx = torch.empty(A), torch.empty(zi), torch.empty(x)
        y = getattr(torch.ops.philtorch, op)(fa, fz, fx)
        assert y.shape == fx.shape and y.is_contiguous()


def test_fake_kernel_rejects_mismatch():
    import philtorch_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        with pytest.raises(RuntimeError):
            torch.ops.philtorch.recur2(torch.empty(5, 99, 2, 2), torch.empty(5, 2), torch.empty(5, 100, 2))


# ------------------------------------------------------------ Python API, CPU route
@pytest.mark.parametrize("unroll", [1, 7, 64])
@pytest.mark.parametrize("shared", [False, True])
def test_lpv_linear_recurrence_cpu_route(unroll, shared):
    from philtorch_amd import lpv

    g = D.rng(10)
    B, T = 3, 301
    a = D.coef(g, (T,) if shared else (B, T), np.float64)
    x, zi = D.normal(g, (B, T), np.float64), D.normal(g, (B,), np.float64)
    y = lpv.linear_recurrence(torch.from_numpy(a), torch.from_numpy(zi), torch.from_numpy(x), unroll_factor=unroll)
    a_full = np.broadcast_to(a, (B, T)) if shared else a
    np.testing.assert_allclose(y.numpy(), oracle.recur(np.ascontiguousarray(a_full), zi, x), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("unroll", [1, 5, 32])
def test_lti_linear_recurrence_cpu_route(unroll):
    from philtorch_amd import lti

    g = D.rng(11)
    B, T = 3, 257
    a = D.coef(g, (B,), np.complex128)
    x, zi = D.normal(g, (B, T), np.complex128), D.normal(g, (B,), np.complex128)
    y = lti.linear_recurrence(torch.from_numpy(a), torch.from_numpy(zi), torch.from_numpy(x), unroll_factor=unroll)
    np.testing.assert_allclose(y.numpy(), oracle.lti_recur(a, zi, x), rtol=1e-10, atol=1e-10)


def test_linear_recurrence_argument_errors():
    from philtorch_amd import lpv, lti

    x = torch.zeros(2, 10)
    with pytest.raises(ValueError):
        lpv.linear_recurrence(torch.zeros(10), torch.zeros(2), x, unroll_factor=0)
    with pytest.raises(ValueError):
        lpv.linear_recurrence(torch.zeros(9), torch.zeros(2), x)
    with pytest.raises(ValueError):
        lpv.linear_recurrence(torch.zeros(10), torch.zeros(3), x)
    with pytest.raises(ValueError):
        lti.linear_recurrence(torch.zeros(3), torch.zeros(2), x)
    with pytest.raises(AssertionError):
        lti.linear_recurrence(torch.zeros(2, 2), torch.zeros(2), x)


def test_extension_flag_and_loader():
    import philtorch_amd

    assert philtorch_amd.EXTENSION_LOADED
    assert philtorch_amd.HELION_LOADED is False
    philtorch_amd.require_extension()


def test_graft_entry_points_importable():
    import __graft_entry__

    assert callable(__graft_entry__.build) and callable(__graft_entry__.smoke)


def test_capi_sosfilt_host_only_calls():
    """Sizes and argument errors of the cascade entry points (nothing launches)."""
    lib = capi.load()
    for dt in (0, 1):
        fwd = lib.phs_sosfilt_workspace_size(dt, 16, 480000, 8, 0)
        bwd = lib.phs_sosfilt_workspace_size(dt, 16, 480000, 8, 1)
        assert 0 < fwd <= bwd
        # one fp64 pair per section and every 32nd step (float32) or every
        # 8th (float64): the gradient backward's lane chunks
        every = 32 if dt == 0 else 8
        assert lib.phs_sosfilt_ckpt_size(dt, 16, 480000, 8) == 16 * 8 * ((480000 + every - 1) // every) * 16
        assert lib.phs_sosfilt_ckpt_size(dt, 3, 100, 2) == 3 * 2 * ((100 + every - 1) // every) * 16
    for bad in ((0, 16, 100, 0), (0, 16, 100, 9), (2, 16, 100, 8), (0, -1, 100, 8)):
        assert lib.phs_sosfilt_workspace_size(*bad, 0) == 0
        assert lib.phs_sosfilt_ckpt_size(*bad) == 0
    d = ctypes.c_void_p(16)
    ws = 1 << 30
    assert lib.phs_sosfilt_fwd(2, 2, 100, 3, d, 0, None, d, d, None, None, d, ws, None) == capi.PHS_ERR_DTYPE
    assert lib.phs_sosfilt_fwd(0, 2, 100, 0, d, 0, None, d, d, None, None, d, ws, None) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_fwd(0, 2, 100, 3, None, 0, None, d, d, None, None, d, ws, None) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_fwd(0, 2, 100, 3, d, 0, None, d, d, None, None, None, 0, None) == capi.PHS_ERR_WORKSPACE
    need = lib.phs_sosfilt_workspace_size(0, 2, 100, 3, 0)
    assert lib.phs_sosfilt_fwd(0, 2, 100, 3, d, 0, None, d, d, None, None, d, need - 1, None) == capi.PHS_ERR_WORKSPACE
    # coefficient gradients need x and the forward's checkpoints
    assert lib.phs_sosfilt_bwd(0, 2, 100, 3, d, 0, None, d, d, None, d, d, None, d, ws, None) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_bwd(1, 2, 100, 3, d, 0, d, None, d, None, d, d, None, d, ws, None) == capi.PHS_ERR_INVALID
    assert lib.phs_sosfilt_fwd(0, 0, 100, 3, None, 0, None, None, None, None, None, None, 0, None) == capi.PHS_OK


def test_capi_filtfilt_host_only_calls():
    """Sizes and argument errors of the zero-phase filter entry point (nothing
    launches)."""
    lib = capi.load()
    for dt, esz in ((0, 4), (1, 8)):
        assert lib.phs_filtfilt_workspace_size(dt, 16, 480000) > 0
        # pass 1's output and its [B, 4] final states
        assert lib.phs_filtfilt_mid_size(dt, 16, 480000) >= 16 * 480000 * esz + 16 * 4 * esz
        # one workspace serves every order: at least the order-4 state-space one
        assert lib.phs_filtfilt_workspace_size(dt, 16, 480000) >= lib.phs_lti_ss_workspace_size(dt, 4, 16, 480000)
    for bad in ((2, 16, 100), (0, -1, 100), (0, 16, 0)):
        assert lib.phs_filtfilt_workspace_size(*bad) == 0
        assert lib.phs_filtfilt_mid_size(*bad) == 0
    d = ctypes.c_void_p(16)
    ws = 1 << 30
    rep = capi.PADMODES["replicate"]

    def call(dt=0, T=100, nb=3, na=2, mode=rep, padlen=9, mid=d, wsb=ws, B=2, b=d):
        return lib.phs_filtfilt_fwd(dt, B, T, b, nb, d, na, 0, mode, padlen, d, d, mid, d, wsb, None)

    assert call(dt=2) == capi.PHS_ERR_DTYPE
    assert call(padlen=100) == capi.PHS_ERR_INVALID  # the reference asserts T > padlen
    assert call(padlen=-1) == capi.PHS_ERR_INVALID
    assert call(T=0, padlen=0) == capi.PHS_ERR_INVALID
    assert call(mode=4) == capi.PHS_ERR_INVALID
    assert call(nb=6) == capi.PHS_ERR_INVALID and call(nb=0) == capi.PHS_ERR_INVALID
    assert call(na=5) == capi.PHS_ERR_INVALID and call(na=0) == capi.PHS_ERR_INVALID
    assert call(mid=None) == capi.PHS_ERR_INVALID and call(b=None) == capi.PHS_ERR_INVALID
    need = lib.phs_filtfilt_workspace_size(0, 2, 100)
    for nb, na in ((3, 2), (2, 1), (5, 4)):
        assert call(wsb=need - 1, nb=nb, na=na) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_filtfilt_fwd(0, 0, 100, None, 3, None, 2, 0, rep, 9, None, None, None, None, 0, None) == capi.PHS_OK


def test_capi_filtfilt_bwd_host_only_calls():
    """Sizes and argument errors of the zero-phase filter's gradients
    (nothing launches)."""
    lib = capi.load()
    for dt, esz in ((0, 4), (1, 8)):
        # dL/dy1 of the interior, three [B, 4] states, the back pad in double
        need = lib.phs_filtfilt_bwd_scratch_size(dt, 2, 16, 480000, 9, 0)
        assert need >= 16 * 480000 * esz + 3 * 16 * 4 * esz + 16 * 9 * 8
        assert lib.phs_filtfilt_bwd_scratch_size(dt, 2, 16, 480000, 100, 0) > need
        # coefficients: pass 1's output, both passes' states [B, T, M], the sums
        coef = lib.phs_filtfilt_bwd_scratch_size(dt, 2, 16, 480000, 9, 1)
        assert coef >= need + 16 * 480000 * esz * (1 + 2 * 2)
        assert lib.phs_filtfilt_bwd_scratch_size(dt, 4, 16, 480000, 9, 1) > coef
    for bad in ((2, 2, 16, 100, 9, 0), (0, 2, -1, 100, 9, 0), (0, 2, 16, -1, 9, 0), (0, 2, 16, 100, -1, 0),
                (0, 0, 16, 100, 9, 0), (0, 5, 16, 100, 9, 1)):
        assert lib.phs_filtfilt_bwd_scratch_size(*bad) == 0
    d = ctypes.c_void_p(16)
    big = 1 << 30
    rep = capi.PADMODES["replicate"]

    def call(dt=0, T=100, nb=3, na=2, mode=rep, padlen=9, sc=d, scb=big, wsb=big, B=2, b=d, gy=d, gx=d, x=d,
             gb=None, ga=None):
        return lib.phs_filtfilt_bwd(dt, B, T, b, nb, d, na, 0, mode, padlen, x, gy, gx, gb, ga, sc, scb, d, wsb,
                                    None)

    assert call(dt=2) == capi.PHS_ERR_DTYPE
    assert call(padlen=100) == capi.PHS_ERR_INVALID
    assert call(padlen=-1) == capi.PHS_ERR_INVALID
    assert call(T=0, padlen=0) == capi.PHS_ERR_INVALID
    assert call(mode=4) == capi.PHS_ERR_INVALID
    assert call(nb=6) == capi.PHS_ERR_INVALID and call(na=0) == capi.PHS_ERR_INVALID
    assert call(b=None) == capi.PHS_ERR_INVALID and call(gy=None) == capi.PHS_ERR_INVALID
    assert call(gx=None) == capi.PHS_ERR_INVALID
    assert call(gb=d) == capi.PHS_ERR_INVALID and call(ga=d) == capi.PHS_ERR_INVALID  # both or neither
    assert call(gb=d, ga=d, x=None) == capi.PHS_ERR_INVALID  # coefficient gradients read x
    need_ws = lib.phs_filtfilt_workspace_size(0, 2, 100)
    for nb, na in ((3, 2), (2, 1), (5, 4)):
        M = max(nb - 1, na)
        need_sc = lib.phs_filtfilt_bwd_scratch_size(0, M, 2, 100, 9, 0)
        need_cf = lib.phs_filtfilt_bwd_scratch_size(0, M, 2, 100, 9, 1)
        assert call(wsb=need_ws - 1, nb=nb, na=na) == capi.PHS_ERR_WORKSPACE
        assert call(scb=need_sc - 1, nb=nb, na=na) == capi.PHS_ERR_WORKSPACE
        assert call(scb=need_cf - 1, nb=nb, na=na, gb=d, ga=d) == capi.PHS_ERR_WORKSPACE
    assert call(sc=None) == capi.PHS_ERR_WORKSPACE
    assert lib.phs_filtfilt_bwd(0, 0, 100, None, 3, None, 2, 0, rep, 9, None, None, None, None, None, None, 0,
                                None, 0, None) == capi.PHS_OK

def test_filtfilt_fused_route_not_taken_on_cpu():
    from philtorch_amd.lti import filtering

    b, a, x = torch.tensor([0.5, 0.2, 0.1]), torch.tensor([-0.5, 0.2]), torch.randn(2, 50)
    assert not filtering._fused_filtfilt_applies(b, a, x, "replicate", "tdf2", {"unroll_factor": 1})


def test_capi_state_space_host_only_calls():
    """Sizes and argument errors of the single-input single-output state space
    and lfilter entry points (nothing launches)."""
    lib = capi.load()
    for dt in (0, 1):
        for M in (1, 2, 3, 4):
            assert lib.phs_lti_ss_workspace_size(dt, M, 16, 480000) > 0
    for bad in ((2, 2, 16, 100), (0, 5, 16, 100), (0, 0, 16, 100), (0, 2, -1, 100)):
        assert lib.phs_lti_ss_workspace_size(*bad) == 0
    d = ctypes.c_void_p(16)
    ws = 1 << 30

    def ss(dt=0, M=3, out_idx=0, a=d):
        return lib.phs_lti_ss_fwd(dt, M, 2, 100, a, 1, None, 0, None, 1, out_idx, None, 0, None, d, d, None, d, ws,
                                  None)

    assert ss(dt=2) == capi.PHS_ERR_DTYPE
    assert ss(M=5) == capi.PHS_ERR_INVALID and ss(out_idx=3) == capi.PHS_ERR_INVALID and ss(a=None) == capi.PHS_ERR_INVALID

    def lf(dt=0, nb=3, na=2, form=0, wsb=ws, b=d):
        return lib.phs_lfilter_fwd(dt, 2, 100, b, nb, d, na, 0, form, None, d, d, None, d, wsb, None)

    assert lf(dt=2) == capi.PHS_ERR_DTYPE
    assert lf(form=2) == capi.PHS_ERR_INVALID
    assert lf(nb=6) == capi.PHS_ERR_INVALID and lf(na=5) == capi.PHS_ERR_INVALID and lf(na=0) == capi.PHS_ERR_INVALID
    assert lf(b=None) == capi.PHS_ERR_INVALID
    assert lf(wsb=lib.phs_lti_ss_workspace_size(0, 2, 2, 100) - 1) == capi.PHS_ERR_WORKSPACE


def test_table_column_detects_only_exact_columns():
    """lfilter's column route (philtorch::biquad_cols) takes b[:, s] of a
    (B, S, 3) table and table[s] of a shared (S, 3) one, by memory
    placement; copies, slices of wider tables, transposed tables, views
    that retain their gradient and tables without a gradient keep the plain
    route."""
    import torch

    from philtorch_amd.lti.filtering import _table_column

    t3 = torch.randn(4, 8, 3, requires_grad=True)
    for s in (0, 5, 7):
        base, col = _table_column(t3[:, s])
        assert base is t3 and col == s
    t2 = torch.randn(8, 2, requires_grad=True)
    base, col = _table_column(t2[3])
    assert base is t2 and col == 3
    assert _table_column(t3[:, 2].clone())[1] == -1
    assert _table_column(t3[:, 2] * 1.0)[1] == -1
    wide = torch.randn(4, 8, 6, requires_grad=True)
    assert _table_column(wide[..., 0:3][:, 1])[1] == -1  # a column of a slice of a wider table
    tt = torch.randn(4, 3, 8, requires_grad=True).transpose(1, 2)  # (4, 8, 3), not the root's layout
    assert _table_column(tt[:, 1])[1] == -1
    v = t3[:, 1]
    v.retain_grad()
    assert _table_column(v)[1] == -1
    assert _table_column(torch.randn(4, 8, 3)[:, 1])[1] == -1  # no gradient wanted
    plain = torch.randn(4, 3, requires_grad=True)
    assert _table_column(plain) == (plain, -1)


def test_lpv_row_scratch_bytes_counts_shared_time_varying_operands():
    """The fused LPV backward's per-row step-gradient scratch: A shared by the
    rows (T, M, M) and b, c, d with one row and T steps count; per-row or
    constant-in-time operands and gradients not wanted do not.  B = 32,
    T = 2^20, M = 4 fp32 (A alone: 2 GiB) is above the limit."""
    import torch

    from philtorch_amd.lpv import ssm

    B, T, M = 32, 1 << 20, 4
    meta = lambda *s: torch.empty(*s, device="meta")  # noqa: E731
    x = meta(B, T)
    need = (True,) * 4
    assert ssm._lpv_row_scratch_bytes(meta(T, M, M), None, None, None, x, need) == B * T * M * M * 4 == 2 << 30
    assert ssm._lpv_row_scratch_bytes(meta(T, M, M), None, None, None, x, need) > ssm._LPV_ROW_SCRATCH_LIMIT
    assert ssm._lpv_row_scratch_bytes(meta(B, T, M, M), None, None, None, x, need) == 0
    assert ssm._lpv_row_scratch_bytes(meta(T, M, M), None, None, None, x, (False, True, True, True)) == 0
    b_step, b_row = meta(1, T, M), meta(B, 1, M)
    d_step = meta(1, T)
    assert ssm._lpv_row_scratch_bytes(meta(B, T, M, M), b_step, b_row, d_step, x, need) == B * T * (M + 1) * 4
    assert ssm._lpv_row_scratch_bytes(meta(B, T, M, M), meta(B, T, M), None, meta(1, 1), x, need) == 0


def test_capi_mimo_state_space_host_only_calls():
    """Sizes and argument errors of the multi-input multi-output state space
    (nothing launches; an empty batch returns at once)."""
    lib = capi.load()
    for dt in (0, 1):
        for M in (1, 2, 3, 4):
            assert lib.phs_mimo_ss_workspace_size(dt, M, 16, 480000) > 0
    for bad in ((2, 2, 16, 100), (0, 5, 16, 100), (0, 0, 16, 100), (0, 2, -1, 100)):
        assert lib.phs_mimo_ss_workspace_size(*bad) == 0
    d = ctypes.c_void_p(16)
    ws = 1 << 30

    def mimo(dt=0, M=2, F=2, P=3, B=2, shared=0, a=d, wsb=ws):
        return lib.phs_mimo_ss_fwd(dt, M, F, P, B, 100, a, d, d, None, shared, None, d, d, None, d, wsb, None)

    assert mimo(dt=2) == capi.PHS_ERR_DTYPE
    for bad in (dict(M=5), dict(M=0), dict(F=0), dict(F=5), dict(P=0), dict(P=5), dict(B=-1), dict(shared=16),
                dict(a=None)):
        assert mimo(**bad) == capi.PHS_ERR_INVALID, bad
    assert mimo(wsb=lib.phs_mimo_ss_workspace_size(0, 2, 2, 100) - 1) == capi.PHS_ERR_WORKSPACE
    assert mimo(B=0) == capi.PHS_OK
    # the coefficient-gradient sums: sizes and argument errors
    assert lib.phs_mimo_ss_grad_sums_scratch_size(0, 16, 480000) >= 16 * 30 * 64 * 8
    assert lib.phs_mimo_ss_grad_sums_scratch_size(2, 16, 100) == 0

    def gsum(dt=0, M=2, F=2, P=3, shared=0, sb=1 << 20, lam=d, gA=d, gD=None, bm=None, gx=None):
        return lib.phs_mimo_ss_grad_sums(dt, M, F, P, 2, 100, lam, d, d, d, bm, None, shared, gA, None, None, gD, gx,
                                         d, sb, None)

    assert gsum(dt=2) == capi.PHS_ERR_DTYPE
    steps, steps_t = capi.PHS_MIMO_A_STEPS, capi.PHS_MIMO_A_STEPS_T
    for bad in (dict(M=0), dict(F=5), dict(P=0), dict(shared=64), dict(lam=None), dict(shared=steps | 1),
                dict(shared=steps_t), dict(shared=steps | steps_t, lam=None), dict(gx=d),
                dict(gx=d, bm=d, lam=None)):
        assert gsum(**bad) == capi.PHS_ERR_INVALID, bad
    assert gsum(sb=8) == capi.PHS_ERR_WORKSPACE
    assert gsum(gA=None) == capi.PHS_OK  # nothing wanted: nothing launched
    # the LPV form: sizes and argument errors
    for dt in (0, 1):
        for M in (1, 2, 3, 4):
            assert lib.phs_lpv_mimo_ss_workspace_size(dt, M, 32, 1 << 20) > 0
    assert lib.phs_lpv_mimo_ss_workspace_size(2, 2, 16, 100) == 0

    def lpv(dt=0, M=2, F=2, P=3, B=2, a_flags=0, shared=0, a=d, wsb=ws):
        return lib.phs_lpv_mimo_ss(dt, M, F, P, B, 100, a, a_flags, d, d, None, shared, None, d, d, None, 0, d, wsb,
                                   None)

    assert lpv(dt=2) == capi.PHS_ERR_DTYPE
    for bad in (dict(M=5), dict(F=0), dict(P=5), dict(B=-1), dict(a_flags=4), dict(shared=1), dict(a=None)):
        assert lpv(**bad) == capi.PHS_ERR_INVALID, bad
    assert lpv(wsb=lib.phs_lpv_mimo_ss_workspace_size(0, 2, 2, 100) - 1) == capi.PHS_ERR_WORKSPACE
    assert lpv(B=0) == capi.PHS_OK


def _mimo_shape_cases(batch, M):
    """(x features or None for 2D x, B, C, D, out_idx) of every branch of the
    reference's B, C and D shape rules that the fused multi-output route
    takes (philtorch/lti/ssm.py:460-485, 513-589)."""
    F, P = 3, 2
    return [
        (F, (M, F), (P, M), (P, F), None),
        (F, (batch, M, F), (batch, P, M), (batch, P, F), None),
        (F, (M, F), (M,), (F,), None),
        (F, (M, F), (batch, M), (batch, F), None),
        (F, (M, F), None, (F,), 1),
        (F, (M, F), (F, M), (), None),
        (M, None, None, None, None),
        (M, None, (P, M), None, None),
        (None, (M,), (P, M), (P,), None),
        (None, (batch, M), (batch, P, M), (batch, P), None),
        (None, (M,), (P, M), None, None),
        (None, (batch, M), None, None, None),
    ]


@pytest.mark.parametrize("case", range(12))
def test_mimo_operands_reproduce_composed_route(case):
    """Each shape case's per-row matrices (lti.ssm._mimo_operands) run through
    the composite of mimo_ss (B x, the scan, the shift, C h + D x) give the
    composed route's y and zf on CPU, for every branch of the reference's
    shape rules the fused route takes."""
    from philtorch_amd.lti import ssm

    batch, N, M = 4, 40, 3  # (batch != M != F: no shape reads two ways)
    F, bs, cs, ds, out_idx = _mimo_shape_cases(batch, M)[case]
    g = torch.Generator().manual_seed(1000 + case)
    rnd = lambda *s: torch.randn(tuple(s), generator=g, dtype=torch.float64)  # noqa: E731
    A = 0.4 * rnd(M, M)
    x = rnd(batch, N) if F is None else rnd(batch, N, F)
    B = None if bs is None else rnd(*bs)
    C = None if cs is None else rnd(*cs)
    D = None if ds is None else rnd(*ds)
    zi = rnd(batch, M)
    ops = ssm._mimo_operands(A, x, B, C, D, out_idx, batch, M)
    assert ops is not None
    x3, Bm, Cm, Dm, vec = ops
    y, zf = ssm._mimo_composite(A, Bm, Cm, Dm, zi, x3)
    y = y.squeeze(-1) if vec else y
    ref, rzf = ssm._state_space(A, x, B, C, D, zi, 1, out_idx, fused=False)
    assert y.shape == ref.shape
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(zf, rzf, rtol=1e-12, atol=1e-12)


def test_mimo_operands_leave_mixed_and_rejected_shapes():
    """Shapes whose reference result broadcasts a one-output term against a
    multi-output one, or that the reference rejects, get no fused operands."""
    from philtorch_amd.lti import ssm

    batch, N, M, F = 4, 10, 2, 3
    A, x = torch.eye(M), torch.randn(batch, N, F)
    assert ssm._mimo_operands(A, x, torch.randn(M, F), torch.randn(M), torch.randn(2, F), None, batch, M) is None
    assert ssm._mimo_operands(A, x, torch.randn(M, F), torch.randn(2, M), torch.randn(F), None, batch, M) is None
    assert ssm._mimo_operands(A, x, torch.randn(M), torch.randn(M), None, None, batch, M) is None
    assert ssm._mimo_operands(A, x, None, torch.randn(M), None, None, batch, M) is None  # B None needs F == M
    assert ssm._mimo_operands(A, x, torch.randn(M, F), torch.randn(M), torch.randn(batch), None, batch, M) is None


def _lpv_mimo_shape_cases(batch, N, M, F, P):
    """(x features or None for 2D x, B, C, D, out_idx) of every branch of the
    reference's LPV B, C and D shape rules with operands constant in time
    that the fused multi-output route takes (philtorch/lpv/ssm.py:413-577)."""
    return [
        (F, (M, F), (P, M), (P, F), None),
        (F, (batch, M, F), (batch, P, M), (batch, P, F), None),
        (F, (M, F), (M,), (F,), None),
        (F, (M, F), (batch, M), (batch, F), None),
        (F, (M, F), None, (F,), 1),
        (F, (M, F), (F, M), (), None),
        (M, None, None, None, None),
        (M, None, (P, M), None, None),
        (None, (M,), (P, M), (P,), None),
        (None, (batch, M), (batch, P, M), (batch, P), None),
        (None, (M,), (P, M), None, None),
        (None, (batch, M), None, None, None),
    ]


@pytest.mark.parametrize("case", range(12))
@pytest.mark.parametrize("shared_A", [False, True])
def test_lpv_mimo_operands_reproduce_composed_route(case, shared_A):
    """Each LPV shape case's matrices (lpv.ssm._lpv_mimo_operands) run
    through the composite of lpv_mimo_ss (B x, the LPV scan, the shift,
    C h + D x) give the composed route's y and zf on CPU."""
    from philtorch_amd.lpv import ssm

    batch, N, M, F, P = 5, 40, 3, 2, 4  # (no two sizes equal: no shape reads two ways)
    Fx, bs, cs, ds, out_idx = _lpv_mimo_shape_cases(batch, N, M, F, P)[case]
    g = torch.Generator().manual_seed(3000 + case)
    rnd = lambda *s: torch.randn(tuple(s), generator=g, dtype=torch.float64)  # noqa: E731
    A = 0.5 * rnd(*((N, M, M) if shared_A else (batch, N, M, M))) / M ** 0.5
    x = rnd(batch, N) if Fx is None else rnd(batch, N, Fx)
    B = None if bs is None else rnd(*bs)
    C = None if cs is None else rnd(*cs)
    D = None if ds is None else rnd(*ds)
    zi = rnd(batch, M)
    ops = ssm._lpv_mimo_operands(x, B, C, D, out_idx, batch, N, M)
    assert ops is not None
    x3, Bm, Cm, Dm, vec = ops
    y, zf = ssm._lpv_mimo_composite(A, Bm, Cm, Dm, zi, x3)
    y = y.squeeze(-1) if vec else y
    ref, rzf = ssm.state_space(A, x, B, C, D, zi=zi, unroll_factor=1, out_idx=out_idx)
    assert y.shape == ref.shape
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(zf, rzf, rtol=1e-12, atol=1e-12)
    # reversed and transposed forms against the composite's definition
    yr, _ = ssm._lpv_mimo_composite(A, Bm, Cm, Dm, zi, x3, reverse=True, transpose_A=True)
    At = A.mT.flip(-3)
    yf, _ = ssm._lpv_mimo_composite(At, Bm, Cm, Dm, zi, x3.flip(1))
    torch.testing.assert_close(yr, yf.flip(1), rtol=1e-12, atol=1e-12)


def test_lpv_mimo_operands_leave_time_varying_and_mixed_shapes():
    """Operands that vary along time, shapes whose one-output term the
    reference broadcasts against a multi-output one, and shapes the reference
    rejects get no fused operands."""
    from philtorch_amd.lpv import ssm

    batch, N, M, F = 5, 40, 3, 2
    x3, x2 = torch.randn(batch, N, F), torch.randn(batch, N)
    o = ssm._lpv_mimo_operands
    assert o(x3, torch.randn(N, M, F), torch.randn(2, M), None, None, batch, N, M) is None  # B (N, M, F)
    assert o(x3, torch.randn(M, F), torch.randn(N, 2, M), None, None, batch, N, M) is None  # C (N, P, M)
    assert o(x2, torch.randn(M), torch.randn(2, M), torch.randn(N), None, batch, N, M) is None  # D (N,)
    assert o(x2, torch.randn(N, M), torch.randn(2, M), None, None, batch, N, M) is None  # B (N, M)
    assert o(x3, torch.randn(M, F), torch.randn(M), torch.randn(2, F), None, batch, N, M) is None  # 1 + 2 outputs
    assert o(x3, torch.randn(M), torch.randn(M), None, None, batch, N, M) is None  # B (M,) with 3D x
