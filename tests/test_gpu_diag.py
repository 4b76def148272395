"""diag_state_space on the GPU with per-channel complex poles (config C2's
law: r ~ U(0.9, 0.999), theta ~ U(0, pi)), through the API, against the
oracle (philtorch/lti/ssm.py:592-833: the B*M scalar recursions run by
LTIRecurrence at :794-804).

A 3D input with one feature per state drives each state channel with its own
signal; with V = I the model is B*M independent scans h[t] = p h[t-1] + x[t],
which oracle.lti_recur computes per channel; the API returns the states
before each step (zi, then h[:-1]) and zf = h[-1].  With a unitary V the
input and initial state are rotated by V^-1 and the states back by V, here
in complex128 around the oracle's scans.  Gradients are checked against the
same API on CPU tensors (the native CPU ops, pinned to the reference's golden
vectors and the oracle's backward in the CPU suite).
"""
import numpy as np
import pytest
import torch

import oracle
from tests import _data as D

pytestmark = pytest.mark.gpu


def _poles(g, shape):
    r = g.uniform(0.9, 0.999, shape)
    th = g.uniform(0, np.pi, shape)
    return (r * np.exp(1j * th)).astype(np.complex64)


def _unitary(g, M):
    q, _ = np.linalg.qr(g.standard_normal((M, M)) + 1j * g.standard_normal((M, M)))
    return q.astype(np.complex64)


def _oracle_diag(L, V, x, zi):
    """States before each step and the final state of the eigenbasis model,
    the scans by the oracle in complex128."""
    B, T, M = x.shape
    Vd = V.astype(np.complex128)
    Vinv = np.linalg.inv(Vd)
    xt = x.astype(np.complex128) @ Vinv.T  # rows x_t -> V^-1 x_t
    zt = zi.astype(np.complex128) @ Vinv.T
    p = L.astype(np.complex128).reshape(B * M)
    xs = np.ascontiguousarray(xt.transpose(0, 2, 1).reshape(B * M, T))
    h = oracle.lti_recur(p, np.ascontiguousarray(zt.reshape(B * M)), xs)
    h = h.reshape(B, M, T).transpose(0, 2, 1) @ Vd.T  # back to the state basis
    y = np.concatenate([zi[:, None, :].astype(np.complex128), h[:, :-1]], axis=1)
    return y, h[:, -1]


@pytest.mark.parametrize("rotated", [False, True], ids=["V=I", "V unitary"])
def test_diag_state_space_per_channel_poles_vs_oracle(hip, rotated):
    from philtorch_amd import lti

    g = D.rng(D.seed_of("diag-c2", rotated))
    B, M, T = 8, 128, 20000  # 1024 channels, as C2
    L = _poles(g, (B, M))
    V = _unitary(g, M) if rotated else np.eye(M, dtype=np.complex64)
    x = D.normal(g, (B, T, M), np.complex64)
    zi = D.normal(g, (B, M), np.complex64)
    print(f"diag_state_space B={B} M={M} T={T} rotated={rotated}", flush=True)
    y, zf = lti.diag_state_space(torch.from_numpy(x).cuda(), L=torch.from_numpy(L).cuda(),
                                 V=torch.from_numpy(V).cuda(), zi=torch.from_numpy(zi).cuda(), unroll_factor=1)
    y_ref, zf_ref = _oracle_diag(L, V, x, zi)
    D.check(y.cpu().numpy(), y_ref, "y", dtype=np.complex64)
    D.check(zf.cpu().numpy(), zf_ref, "zf", dtype=np.complex64, scale=np.max(np.abs(y_ref)))


@pytest.mark.parametrize("rotated", [False, True], ids=["V=I", "V unitary"])
def test_diag_state_space_gradients_vs_cpu_route(hip, rotated):
    from philtorch_amd import lti

    g = D.rng(D.seed_of("diag-c2-grad", rotated))
    B, M, T = 4, 16, 6000
    L = _poles(g, (B, M))
    V = _unitary(g, M) if rotated else np.eye(M, dtype=np.complex64)
    x = D.normal(g, (B, T, M), np.complex64)
    zi = D.normal(g, (B, M), np.complex64)
    gy = D.normal(g, (B, T, M), np.complex64)
    grads = []
    for dev in ("cuda", "cpu"):
        tL = torch.tensor(L, device=dev, requires_grad=True)
        tx = torch.tensor(x, device=dev, requires_grad=True)
        tz = torch.tensor(zi, device=dev, requires_grad=True)
        y, _ = lti.diag_state_space(tx, L=tL, V=torch.tensor(V, device=dev), zi=tz, unroll_factor=1)
        (y * torch.tensor(gy, device=dev).conj()).real.sum().backward()
        grads.append([t.grad.cpu().numpy() for t in (tL, tx, tz)])
    for name, got, ref in zip(("grad_L", "grad_x", "grad_zi"), *grads):
        D.check(got, ref, name, dtype=np.complex64)
