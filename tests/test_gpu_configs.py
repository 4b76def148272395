"""Parity at the benchmark's own workloads: every BASELINE config, at its full
shape and with its own input law, built by bench.py's workload classes (the
exact tensors the bench times), checked against the oracle.

* C1  LPV scalar fp32, B=64, T=65536: every row, forward and backward.
* C5  LPV scalar, a = 0.999 tanh(2 z), B=8, T=2^24 (about 16k look-back tiles
      per pass in fp64): every row, forward and backward, in fp32 (1e-4) and
      fp64 (1e-10 of max|ref|, the north star's bar).
* C2  LTI complex64 diagonal scan, C=1024 channels, T=262144, poles of radius
      up to 0.999: the GPU runs all channels, the oracle checks 16 of them
      (the signal is drawn on the GPU: a CPU draw of 2^29 normals is slow).
* C3  LPV 2x2 fp32, B=32, T=2^20 (683 look-back tiles per row): all rows on
      the GPU, three checked.
* C4  the 8-section SOS cascade, B=16, T=480000: op level (one lti_recur2 and
      its backward per section, every section's gradients), fused (sosfilt)
      and the caller pattern (8 x lti.lfilter + autograd w.r.t. x, b, a),
      two rows checked.

The oracle restates the reference CPU loops (philtorch/csrc/host_recurN.cpp:
81-111, host_lti_recur.cpp:4-80, host_lti_recurN.cpp:4-108) and the backward
closures (philtorch/__init__.py:34-148).  The bar is BASELINE's:
max|d| <= 1e-4 max|ref| (fp32, complex64), 1e-10 max|ref| (fp64).
"""
import numpy as np
import pytest

from tests import _data as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bench_mod(hip):
    import bench

    return bench


def _np(t):
    return t.detach().cpu().numpy()


def _free():
    import gc

    import torch

    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["c1", "c5", "c5_f64"])
def test_lpv_scalar_config(bench_mod, name):
    import oracle

    w = bench_mod.make_workload(name)
    print(f"[{name}] B={w.B} T={w.T} {w.dtype_tag}", flush=True)
    y = w.step_fwd()
    gA, gzi, gx = w.step_bwd(y)
    got = [_np(v) for v in (y, gA, gzi, gx)]
    del y, gA, gzi, gx
    w.dev = None
    _free()
    a, x, y0, gy = (v.numpy() for v in w.cpu)
    y_ref = oracle.recur(a, y0, x)
    D.check(got[0], y_ref, f"{name} y")
    refs = oracle.recur_bwd(a, y0, y_ref, gy)
    for nm, g, r in zip(("grad_a", "grad_y0", "grad_x"), got[1:], refs):
        D.check(g, r, f"{name} {nm}")


def test_c2_config(hip):
    """C2's law at its shape.  The 2^29 complex normals of x and the upstream
    gradient are drawn on the GPU (seeded; a CPU draw of that size takes
    minutes), the poles and initial states on the CPU as the bench draws
    them; the oracle checks 16 channels copied back."""
    import torch

    import oracle

    C, T = 1024, 262144
    print(f"[c2] C={C} T={T} c64", flush=True)
    g = torch.Generator().manual_seed(2)
    r = torch.rand(C, generator=g, dtype=torch.float64) * 0.099 + 0.9
    th = torch.rand(C, generator=g, dtype=torch.float64) * torch.pi
    p = torch.polar(r, th).to(torch.complex64)
    zi = torch.complex(torch.randn(C, generator=g), torch.randn(C, generator=g))
    gd = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(C, T, generator=gd, dtype=torch.complex64, device="cuda")
    gy = torch.randn(C, T, generator=gd, dtype=torch.complex64, device="cuda")
    pd, zid = p.cuda(), zi.cuda()
    rows = np.unique(np.concatenate([np.arange(0, C, 67), [C - 1]])).tolist()
    y = torch.ops.philtorch.lti_recur(pd, zid, x)
    gp, gzi, gx = torch.ops.philtorch.lti_recur_backward(pd, zid, y, gy)
    got = [_np(y[rows]), _np(gp[rows]), _np(gzi[rows]), _np(gx[rows])]
    xs, gys = _np(x[rows]), _np(gy[rows])
    del y, gp, gzi, gx, x, gy
    _free()
    ps, zs = p.numpy()[rows], zi.numpy()[rows]
    y_ref = oracle.lti_recur(ps, zs, xs)
    D.check(got[0], y_ref, "c2 y")
    refs = oracle.lti_recur_bwd(ps, zs, y_ref, gys)
    for nm, gg, rf in zip(("grad_p", "grad_zi", "grad_x"), got[1:], refs):
        D.check(gg, rf, f"c2 {nm}")


def test_c3_config(bench_mod):
    import oracle

    w = bench_mod.make_workload("c3")
    print(f"[c3] B={w.B} T={w.T} f32 2x2", flush=True)
    rows = [0, 13, w.B - 1]
    y = w.step_fwd()
    gA, gzi, gx = w.step_bwd(y)
    got = [_np(y[rows]), _np(gA[rows]), _np(gzi[rows]), _np(gx[rows])]
    del y, gA, gzi, gx
    w.dev = None
    _free()
    A, x, zi, gy = (np.ascontiguousarray(v.numpy()[rows]) for v in w.cpu)
    y_ref = oracle.recurN(A, zi, x)
    D.check(got[0], y_ref, "c3 y")
    refs = oracle.recurN_bwd(A, zi, y_ref, gy)
    for nm, g, rf in zip(("grad_A", "grad_zi", "grad_x"), got[1:], refs):
        D.check(g, rf, f"c3 {nm}")


def test_c4_op_level_config(bench_mod):
    """The op-level cascade: section s scans section s-1's output; the
    backward runs the sections in reverse, each returning its own grad_A."""
    import torch

    import oracle

    w = bench_mod.make_workload("c4")
    print(f"[c4] B={w.B} T={w.T} S={w.S} f32", flush=True)
    rows = [0, w.B - 1]
    ys = w.step_fwd()
    _, _, zi, gy = w.dev
    g = gy
    gAs = [None] * w.S
    gzis = [None] * w.S
    for s in reversed(range(w.S)):
        gAs[s], gzis[s], g = torch.ops.philtorch.lti_recurN_backward(w.A_sec[s], zi, ys[s], g)
    got_y = [_np(ys[s][rows]) for s in range(w.S)]
    got_gA = [_np(gAs[s][rows]) for s in range(w.S)]
    got_gzi = [_np(gzis[s][rows]) for s in range(w.S)]
    got_gx = _np(g[rows])
    del ys, g, gAs, gzis
    w.dev = None
    _free()
    A, x, zi, gy = (v.numpy() for v in w.cpu)
    A, x, zi, gy = A[rows], np.ascontiguousarray(x[rows]), zi[rows], np.ascontiguousarray(gy[rows])
    h, y_ref = x, []
    for s in range(w.S):
        h = oracle.lti_recurN(np.ascontiguousarray(A[:, s]), zi, h)
        y_ref.append(h)
        D.check(got_y[s], h, f"c4 y section {s}")
    g = gy
    for s in reversed(range(w.S)):
        gA, gz, g = oracle.lti_recurN_bwd(np.ascontiguousarray(A[:, s]), zi, y_ref[s], g)
        D.check(got_gA[s], gA, f"c4 grad_A section {s}")
        D.check(got_gzi[s], gz, f"c4 grad_zi section {s}")
    D.check(got_gx, g, "c4 grad_x")


def test_c4_fused_config(bench_mod):
    """The fused cascade on the C4 signal and sections: forward and the
    gradients w.r.t. x and every section's coefficients, against the
    oracle's per-section chain evaluated in fp64 on the same fp32 inputs (a
    high-gain 8-section fp32 chain carries rounding of the order of the bar
    in its own coefficient gradients)."""
    import oracle

    w = bench_mod.make_workload("c4_fused")
    print(f"[c4_fused] B={w.B} T={w.T} S={w.S} f32", flush=True)
    rows = [0, w.B - 1]
    out = w.step_fwd()
    gx, gsos, gzi = w.step_bwd(out)
    got = [_np(out[0][rows]), _np(gx[rows]), _np(gsos[rows])]
    del out, gx, gsos, gzi
    w.dev = None
    _free()
    sos, x, gy = (np.ascontiguousarray(v.numpy()[rows]).astype(np.float64) for v in w.cpu)
    y_ref, _ = oracle.sosfilt(sos, x)
    gsos_ref, _, gx_ref = oracle.sosfilt_bwd(sos, x, None, gy)
    gsos_ref[..., 3] = 0.0
    D.check(got[0], y_ref, "c4_fused y", dtype=np.float32)
    D.check(got[1], gx_ref, "c4_fused grad_x", dtype=np.float32)
    D.check(got[2], gsos_ref, "c4_fused grad_sos", dtype=np.float32)


def test_c4_api_config(bench_mod):
    """The C4 caller pattern exactly as the bench times it, ``for s in
    range(8): y = lti.lfilter(b[:, s], a[:, s], y, form="tdf2",
    unroll_factor=1)`` at B=16, T=480000 (every call the biquad kernels),
    then autograd w.r.t. x, b and a; two rows against the oracle's
    per-section chain evaluated in fp64 on the same fp32 inputs
    (philtorch/lti/filtering.py:211-333 per call)."""
    import oracle

    w = bench_mod.make_workload("c4_api")
    print(f"[c4_api] B={w.B} T={w.T} S={w.S} f32", flush=True)
    rows = [0, w.B - 1]
    out = w.step_fwd()
    gx, gb, ga = w.step_bwd(out)
    got = [_np(out[0][rows]), _np(gx[rows]), _np(gb[rows]), _np(ga[rows])]
    del out, gx, gb, ga
    w.dev = None
    _free()
    sos, x, gy = (np.ascontiguousarray(v.numpy()[rows]).astype(np.float64) for v in w.cpu)
    y_ref, _ = oracle.sosfilt(sos, x)
    gsos_ref, _, gx_ref = oracle.sosfilt_bwd(sos, x, None, gy)
    D.check(got[0], y_ref, "c4_api y", dtype=np.float32)
    D.check(got[1], gx_ref, "c4_api grad_x", dtype=np.float32)
    D.check(got[2], gsos_ref[..., 0:3], "c4_api grad_b", dtype=np.float32)
    D.check(got[3], gsos_ref[..., 4:6], "c4_api grad_a", dtype=np.float32)
