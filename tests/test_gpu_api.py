"""The Python API on its native route (HIP kernels) and the autograd contract.

* native route == pure-PyTorch route for the scans, lfilter/filtfilt (the SOS
  composition of config 4), state_space and diag_state_space (config 2's call);
* gradcheck, gradgradcheck and forward-mode AD through the Function wrappers
  and the registered ops, fp64 and complex128 (reference tests/test_grad.py);
* torch.library.opcheck on every op (reference tests/test_pt2_comp.py);
* fused backward == composite backward at sizes with many tiles.
"""
import numpy as np
import pytest
import torch

from tests import _data as D

pytestmark = pytest.mark.gpu


def _pair(x):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t, t.cuda()


def _close(got, ref, dtype, name=""):
    D.check(got.detach().cpu().numpy(), ref.detach().cpu().numpy(), name, dtype=np.dtype(dtype))


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.complex64])
def test_linear_recurrence_native_equals_loop(hip, dtype):
    from philtorch_amd import lpv, lti

    g = D.rng(D.seed_of("api-lr", np.dtype(dtype).str))
    B, T = 3, 3000
    a_c, a_g = _pair(D.coef(g, (B, T), dtype))
    z_c, z_g = _pair(D.normal(g, (B,), dtype))
    x_c, x_g = _pair(D.normal(g, (B, T), dtype))
    _close(lpv.linear_recurrence(a_g, z_g, x_g), lpv.linear_recurrence(a_c, z_c, x_c, unroll_factor=50), dtype)
    l_c, l_g = _pair(D.coef(g, (B,), dtype))
    from philtorch_amd.lti import LTIRecurrence

    _close(LTIRecurrence.apply(l_g, z_g, x_g), lti.linear_recurrence(l_c, z_c, x_c, unroll_factor=50), dtype)


@pytest.mark.parametrize("form", ["tdf2", "df2"])
def test_lfilter_sos_cascade_native_equals_cpu(hip, form):
    from philtorch_amd import lti

    g = D.rng(31)
    B, S, T = 4, 8, 20000
    r, th = g.uniform(0.5, 0.98, (B, S)), g.uniform(0, np.pi, (B, S))
    a = np.stack([-2 * r * np.cos(th), r * r], -1)
    rz, thz = g.uniform(0, 1.2, (B, S)), g.uniform(0, np.pi, (B, S))
    b = np.stack([np.ones((B, S)), -2 * rz * np.cos(thz), rz * rz], -1)
    x = g.standard_normal((B, T))
    yc, yg = torch.from_numpy(x), torch.from_numpy(x).cuda()
    for s in range(S):
        bs, as_ = torch.from_numpy(b[:, s]), torch.from_numpy(a[:, s])
        yc = lti.lfilter(bs, as_, yc, form=form, unroll_factor=1)
        yg = lti.lfilter(bs.cuda(), as_.cuda(), yg, form=form, unroll_factor=1)
    _close(yg, yc, np.float64, "sos cascade")
    bs, as_ = torch.from_numpy(b[:, 0]), torch.from_numpy(a[:, 0])
    _close(lti.filtfilt(bs.cuda(), as_.cuda(), torch.from_numpy(x).cuda(), unroll_factor=1),
           lti.filtfilt(bs, as_, torch.from_numpy(x), unroll_factor=1), np.float64, "filtfilt")


def test_lfilter_fp32_native_vs_fp64(hip):
    """fp32 native biquad cascade (config 4 numerics) vs the fp64 CPU route."""
    from philtorch_amd import lti

    g = D.rng(32)
    B, S, T = 2, 8, 50000
    r, th = g.uniform(0.5, 0.98, (B, S)), g.uniform(0, np.pi, (B, S))
    a = np.stack([-2 * r * np.cos(th), r * r], -1)
    rz, thz = g.uniform(0, 1.2, (B, S)), g.uniform(0, np.pi, (B, S))
    b = np.stack([np.ones((B, S)), -2 * rz * np.cos(thz), rz * rz], -1)
    x = g.standard_normal((B, T))
    y64, y32 = torch.from_numpy(x), torch.from_numpy(x).float().cuda()
    for s in range(S):
        y64 = lti.lfilter(torch.from_numpy(b[:, s]), torch.from_numpy(a[:, s]), y64, unroll_factor=1)
        y32 = lti.lfilter(torch.from_numpy(b[:, s]).float().cuda(), torch.from_numpy(a[:, s]).float().cuda(), y32,
                          unroll_factor=1)
    D.check(y32.cpu().double().numpy(), y64.numpy(), "fp32 cascade", dtype=np.float32)


def test_state_space_lpv_native_equals_cpu(hip):
    from philtorch_amd import lpv

    g = D.rng(33)
    B, T = 3, 7000
    A = D.biquad_A(g, (B, T), np.float64)
    x = D.normal(g, (B, T), np.float64)
    zi = D.normal(g, (B, 2), np.float64)
    C = np.array([0.4, -1.1])
    args_c = [torch.from_numpy(v) for v in (A, x)]
    args_g = [v.cuda() for v in args_c]
    yc, zc = lpv.state_space(*args_c, C=torch.from_numpy(C), zi=torch.from_numpy(zi), unroll_factor=1)
    yg, zg = lpv.state_space(*args_g, C=torch.from_numpy(C).cuda(), zi=torch.from_numpy(zi).cuda(), unroll_factor=1)
    _close(yg, yc, np.float64, "y")
    _close(zg, zc, np.float64, "zf")


def test_state_space_lti_order3_native_equals_cpu(hip):
    """A third-order LTI system through state_space: native order-M scan on
    the GPU, the reference's pure-PyTorch route on the CPU."""
    from philtorch_amd import lti

    g = D.rng(34)
    B, T = 3, 5000
    A = D.stable_matrix(g, (), 3, np.float64)
    x = D.normal(g, (B, T), np.float64)
    zi = D.normal(g, (B, 3), np.float64)
    Bm = np.array([1.0, -0.5, 0.25])
    C = np.array([0.4, -1.1, 0.7])
    yc, zc = lti.state_space(torch.from_numpy(A), torch.from_numpy(x), B=torch.from_numpy(Bm), C=torch.from_numpy(C),
                             zi=torch.from_numpy(zi), unroll_factor=1)
    yg, zg = lti.state_space(torch.from_numpy(A).cuda(), torch.from_numpy(x).cuda(), B=torch.from_numpy(Bm).cuda(),
                             C=torch.from_numpy(C).cuda(), zi=torch.from_numpy(zi).cuda(), unroll_factor=1)
    _close(yg, yc, np.float64, "y")
    _close(zg, zc, np.float64, "zf")


def test_diag_state_space_complex_native_equals_cpu(hip):
    """Config 2's call: per-channel complex poles through LTIRecurrence."""
    from philtorch_amd import lti

    g = D.rng(34)
    C_, T = 64, 5000
    p = (g.uniform(0.9, 0.999, C_) * np.exp(1j * g.uniform(0, np.pi, C_))).astype(np.complex64)
    x = D.normal(g, (C_, T), np.complex64)
    zi = D.normal(g, (C_, 1), np.complex64)
    L = torch.from_numpy(p)
    yc, zc = lti.diag_state_space(torch.from_numpy(x), L=L[:1] * 0 + L[0], zi=torch.from_numpy(zi[:, :1]), unroll_factor=1)
    yg, zg = lti.diag_state_space(torch.from_numpy(x).cuda(), L=(L[:1] * 0 + L[0]).cuda(),
                                  zi=torch.from_numpy(zi[:, :1]).cuda(), unroll_factor=1)
    _close(yg, yc, np.complex64, "y")


# ------------------------------------------------------------ autograd contract
def _grad_inputs(g, kind, dtype, B=3, T=11, shared=False):
    dev = "cuda"
    if kind == "lpv":
        A = D.coef(g, (T,) if shared else (B, T), dtype)
        zi, x = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype)
    elif kind == "lti":
        A = D.coef(g, (1,) if shared else (B,), dtype)
        zi, x = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype)
    elif kind == "lpv2":
        A = D.biquad_A(g, (T,) if shared else (B, T), dtype)
        zi, x = D.normal(g, (B, 2), dtype), D.normal(g, (B, T, 2), dtype)
    elif kind == "lti2":
        A = D.biquad_A(g, () if shared else (B,), dtype)
        zi, x = D.normal(g, (B, 2), dtype), D.normal(g, (B, T, 2), dtype)
    elif kind == "lpv3":  # order-M kernels (M = 3, 4)
        A = D.stable_matrix(g, (T,) if shared else (B, T), 3, dtype)
        zi, x = D.normal(g, (B, 3), dtype), D.normal(g, (B, T, 3), dtype)
    else:  # lti4
        A = D.stable_matrix(g, () if shared else (B,), 4, dtype)
        zi, x = D.normal(g, (B, 4), dtype), D.normal(g, (B, T, 4), dtype)
    return [torch.from_numpy(np.ascontiguousarray(v)).to(dev).requires_grad_(True) for v in (A, zi, x)]


def _fn(kind):
    from philtorch_amd.lpv import MatrixRecurrence
    from philtorch_amd.lti import LTIMatrixRecurrence, LTIRecurrence

    return {
        "lpv": torch.ops.philtorch.recur,
        "lti": LTIRecurrence.apply,
        "lpv2": MatrixRecurrence.apply,
        "lti2": LTIMatrixRecurrence.apply,
        "lpv3": MatrixRecurrence.apply,
        "lti4": LTIMatrixRecurrence.apply,
    }[kind]


@pytest.mark.parametrize("kind", ["lpv", "lti", "lpv2", "lti2", "lpv3", "lti4"])
@pytest.mark.parametrize("dtype", [np.float64, np.complex128])
@pytest.mark.parametrize("shared", [False, True])
def test_gradcheck_gradgradcheck(hip, kind, dtype, shared):
    g = D.rng(D.seed_of("grad", kind, np.dtype(dtype).str, shared))
    inputs = _grad_inputs(g, kind, dtype, shared=shared)
    f = _fn(kind)
    fwd_ad = kind != "lpv"  # register_autograd ops have no forward-mode formula
    assert torch.autograd.gradcheck(f, inputs, check_forward_ad=fwd_ad)
    assert torch.autograd.gradgradcheck(f, inputs, check_fwd_over_rev=fwd_ad)


@pytest.mark.parametrize("op,kind", [("recur", "lpv"), ("recur2", "lpv2"), ("recurN", "lpv2"), ("recurN", "lpv3"),
                                     ("lti_recur", "lti"), ("lti_recur2", "lti2"), ("lti_recurN", "lti2"),
                                     ("lti_recurN", "lti4")])
def test_opcheck(hip, op, kind):
    g = D.rng(D.seed_of("opcheck", op, kind))
    A, zi, x = _grad_inputs(g, kind, np.float64, B=2, T=40)
    torch.library.opcheck(getattr(torch.ops.philtorch, op), (A, zi, x))


@pytest.mark.parametrize("kind", ["lpv", "lti", "lpv2", "lti2", "lpv3", "lti4"])
def test_fused_backward_equals_composite(hip, kind):
    """Large enough for many tiles: the fused kernel (no create_graph) and the
    composite formula (create_graph) give the same gradients."""
    g = D.rng(D.seed_of("fused", kind))
    A, zi, x = _grad_inputs(g, kind, np.float64, B=3, T=40000)
    f = _fn(kind)
    y = f(A, zi, x)
    gy = torch.randn_like(y)
    fused = torch.autograd.grad(y, (A, zi, x), gy, retain_graph=True)
    comp = torch.autograd.grad(y, (A, zi, x), gy, create_graph=True)
    for a_, b_, n in zip(fused, comp, ("A", "zi", "x")):
        D.check(a_.detach().cpu().numpy(), b_.detach().cpu().numpy(), n, dtype=np.float64)
