"""The philtorch-style Python API on its pure-PyTorch route (CPU tensors).

Pins the host logic that sits around the native scans: companion-form
realisation, state shifting, B/C/D handling, zi/zf streaming, filtfilt padding
and the blocked fallbacks, against SciPy (the reference's own test oracle,
philtorch tests/test_lti_lfilter.py) and against each other.
"""
import numpy as np
import pytest
import scipy.signal
import torch

from philtorch_amd import lpv, lti
from philtorch_amd.mat import companion
from tests import _data as D


def _biquads(g, n):
    r = g.uniform(0.5, 0.95, n)
    th = g.uniform(0, np.pi, n)
    a = np.stack([-2 * r * np.cos(th), r * r], -1)
    rz = g.uniform(0, 1.2, n)
    thz = g.uniform(0, np.pi, n)
    b = np.stack([np.ones(n), -2 * rz * np.cos(thz), rz * rz], -1)
    return b, a


def test_companion():
    a = torch.tensor([[0.5, -0.25, 0.1]])
    A = companion(a)[0]
    np.testing.assert_allclose(A.numpy(), [[-0.5, 0.25, -0.1], [1, 0, 0], [0, 1, 0]])


@pytest.mark.parametrize("form", ["tdf2", "df2"])
@pytest.mark.parametrize("unroll", [None, 1, 9])
def test_lfilter_matches_scipy(form, unroll):
    g = D.rng(20)
    b, a = _biquads(g, 3)
    x = g.standard_normal((3, 300))
    y = lti.lfilter(torch.from_numpy(b), torch.from_numpy(a), torch.from_numpy(x), form=form, unroll_factor=unroll)
    for i in range(3):
        ref = scipy.signal.lfilter(b[i], np.r_[1.0, a[i]], x[i])
        np.testing.assert_allclose(y[i].numpy(), ref, rtol=1e-10, atol=1e-10)


def test_lfilter_zi_zf_streaming_matches_scipy():
    g = D.rng(21)
    b, a = _biquads(g, 2)
    x = g.standard_normal((2, 400))
    zi = g.standard_normal((2, 2))
    y, zf = lti.lfilter(torch.from_numpy(b), torch.from_numpy(a), torch.from_numpy(x), zi=torch.from_numpy(zi),
                        unroll_factor=1)
    for i in range(2):
        ref, zf_ref = scipy.signal.lfilter(b[i], np.r_[1.0, a[i]], x[i], zi=zi[i])
        np.testing.assert_allclose(y[i].numpy(), ref, rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(zf[i].numpy(), zf_ref, rtol=1e-10, atol=1e-10)
    # chunked continuation equals one pass (philtorch tests/test_lpv_filters.py:394-418)
    tb, ta = torch.from_numpy(b), torch.from_numpy(a)
    y1, z1 = lti.lfilter(tb, ta, torch.from_numpy(x[:, :150]), zi=torch.from_numpy(zi), unroll_factor=1)
    y2, z2 = lti.lfilter(tb, ta, torch.from_numpy(x[:, 150:]), zi=z1, unroll_factor=1)
    np.testing.assert_allclose(torch.cat([y1, y2], 1).numpy(), y.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(z2.numpy(), zf.numpy(), rtol=1e-12, atol=1e-12)


def test_lfilter_zi_matches_scipy():
    g = D.rng(22)
    b, a = _biquads(g, 4)
    zi = lti.lfilter_zi(torch.from_numpy(a), torch.from_numpy(b))
    for i in range(4):
        np.testing.assert_allclose(zi[i].numpy(), scipy.signal.lfilter_zi(b[i], np.r_[1.0, a[i]]), rtol=1e-10)


def test_filtfilt_matches_scipy():
    g = D.rng(23)
    b, a = _biquads(g, 2)
    x = g.standard_normal((2, 500))
    y = lti.filtfilt(torch.from_numpy(b), torch.from_numpy(a), torch.from_numpy(x), unroll_factor=1)
    for i in range(2):
        # philtorch pads by edge replication (padmode="replicate"); compare against
        # SciPy on the same replicated extension with padlen 0
        edge = 9
        ext = np.r_[np.full(edge, x[i, 0]), x[i], np.full(edge, x[i, -1])]
        ref = scipy.signal.filtfilt(b[i], np.r_[1.0, a[i]], ext, padlen=0)[edge:-edge]
        np.testing.assert_allclose(y[i].numpy(), ref, rtol=1e-9, atol=1e-9)


def test_sos_cascade_matches_scipy_sosfilt():
    g = D.rng(24)
    b, a = _biquads(g, 4)  # one batch item, 4 sections
    x = g.standard_normal(600)
    y = torch.from_numpy(x)[None]
    for s in range(4):
        y = lti.lfilter(torch.from_numpy(b[s]), torch.from_numpy(a[s]), y, unroll_factor=1)
    sos = np.concatenate([b, np.c_[np.ones(4), a]], axis=1)
    np.testing.assert_allclose(y[0].numpy(), scipy.signal.sosfilt(sos, x), rtol=1e-9, atol=1e-9)


def test_sosfilt_cpu_route_matches_scipy():
    """lti.sosfilt on CPU tensors (one lfilter(tdf2) per section), scipy's
    layout of zi/zf, a0 normalisation, 1D and 2D inputs."""
    g = D.rng(25)
    sos = D.sos_coefs(g, (), 3, np.float64)
    sos[1] *= 2.0  # a0 = 2 for one section
    x = g.standard_normal((2, 400))
    zi = g.standard_normal((3, 2, 2))
    y, zf = lti.sosfilt(torch.from_numpy(sos), torch.from_numpy(x), zi=torch.from_numpy(zi))
    sos_n = sos / sos[:, 3:4]  # scipy takes normalised sections only
    ry, rzf = scipy.signal.sosfilt(sos_n, x, axis=-1, zi=zi)
    np.testing.assert_allclose(y.numpy(), ry, rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(zf.numpy(), rzf, rtol=1e-9, atol=1e-9)
    y1 = lti.sosfilt(torch.from_numpy(sos), torch.from_numpy(x[0]))
    np.testing.assert_allclose(y1.numpy(), scipy.signal.sosfilt(sos_n, x[0]), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("unroll", [1, 4, 13])
@pytest.mark.parametrize("batched", [False, True])
def test_lti_state_space_recursion_unrolled_equals_loop(unroll, batched):
    g = D.rng(25)
    B, T = 3, 101
    A = torch.from_numpy(D.biquad_A(g, (B,) if batched else (), np.float64))
    zi, x = torch.from_numpy(D.normal(g, (B, 2), np.float64)), torch.from_numpy(D.normal(g, (B, T, 2), np.float64))
    ref = lti.state_space_recursion(A, zi, x, unroll_factor=1)
    got = lti.state_space_recursion(A, zi, x, unroll_factor=unroll)
    np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=1e-10, atol=1e-10)
    got0 = lti.state_space_recursion(A, zi, x[..., 0], unroll_factor=unroll, out_idx=0)
    ref0 = lti.state_space_recursion(A, zi, torch.stack([x[..., 0], torch.zeros_like(x[..., 0])], -1))[..., 0]
    np.testing.assert_allclose(got0.numpy(), ref0.numpy(), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("unroll", [1, 5, 16])
@pytest.mark.parametrize("shared", [False, True])
def test_lpv_state_space_recursion_unrolled_matches_oracle(unroll, shared):
    import oracle

    g = D.rng(26)
    B, T = 2, 77
    A = D.biquad_A(g, (T,) if shared else (B, T), np.float64)
    zi, x = D.normal(g, (B, 2), np.float64), D.normal(g, (B, T, 2), np.float64)
    got = lpv.state_space_recursion(torch.from_numpy(A), torch.from_numpy(zi), torch.from_numpy(x),
                                    unroll_factor=unroll)
    np.testing.assert_allclose(got.numpy(), oracle.recurN(A, zi, x), rtol=1e-10, atol=1e-10)


def test_lpv_equals_lti_for_constant_coefficients():
    """philtorch tests/test_lpv_ssm.py:27-54: time-constant LPV == LTI."""
    g = D.rng(27)
    B, T = 2, 64
    A = torch.from_numpy(D.biquad_A(g, (B,), np.float64))
    x = torch.from_numpy(D.normal(g, (B, T), np.float64))
    C = torch.tensor([0.3, -0.7], dtype=torch.float64)
    Bm = torch.tensor([1.0, 0.5], dtype=torch.float64)
    y_lti = lti.state_space(A, x, B=Bm, C=C, D=torch.tensor(0.2, dtype=torch.float64), unroll_factor=1)
    y_lpv = lpv.state_space(A.unsqueeze(1).expand(B, T, 2, 2), x, B=Bm, C=C, D=torch.tensor(0.2, dtype=torch.float64),
                            unroll_factor=1)
    np.testing.assert_allclose(y_lpv.numpy(), y_lti.numpy(), rtol=1e-12, atol=1e-12)


def test_diag_state_space_matches_state_space():
    g = D.rng(28)
    B, T = 2, 80
    A = torch.from_numpy(D.biquad_A(g, (), np.float64))
    x = torch.from_numpy(D.normal(g, (B, T), np.float64))
    C = torch.tensor([0.3, -0.7], dtype=torch.float64)
    zi = torch.from_numpy(D.normal(g, (B, 2), np.float64))
    y_ref, zf_ref = lti.state_space(A, x, C=C, zi=zi, unroll_factor=1)
    y, zf = lti.diag_state_space(x, A=A, C=C, zi=zi, unroll_factor=1)
    np.testing.assert_allclose(y.real.numpy(), y_ref.numpy(), rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(zf.real.numpy(), zf_ref.numpy(), rtol=1e-9, atol=1e-9)
