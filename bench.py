#!/usr/bin/env python3
"""Throughput of the linear-recurrence core, forward + backward, on one MI355X.

Default workload (the metric's config): the
first-order LPV scan, a[B,T]~U(-0.99,0.99), x[B,T]~N(0,1), y0[B]~N(0,1),
upstream grad g[B,T]~N(0,1), B=64, T=65536, fp32, generated on the CPU with
torch.Generator().manual_seed(1) and copied to the GPU before timing.  The
other BASELINE configs run with --config c2|c3|c4|c5|c5_f64 (same output
format, their own metric string).

One step = the hot path over one batch: the forward scan op and the fused
adjoint op (grads w.r.t. the coefficients, the input and the initial state):
  c1, c5  philtorch::recur + recur_backward                 (LPV scalar)
  c2      philtorch::lti_recur + lti_recur_backward         (LTI scalar, complex64)
  c3      philtorch::recur2 + recurN_backward               (LPV 2x2)
  c3_lpv_ss  lpv.state_space of a time-varying biquad (tdf2, one output), forward only (philtorch::lpv_ss)
  c3_lpv_ss_grad  the same plus gradients w.r.t. x and zi (a reversed lpv_ss pass over the adjoint model)
  c3_lpv_ss_coef  the same plus gradients w.r.t. A[t], b[t], d[t] too (philtorch::lpv_ss_states forward,
                  philtorch::lpv_ss_backward given its states)
  c4      8 x (philtorch::lti_recur2 + lti_recurN_backward) (LTI biquad cascade)
  c4_fused  philtorch::sosfilt + sosfilt_backward              (the same cascade, fused)
  c4_api  8 x lti.lfilter(tdf2, unroll_factor=1) + autograd   (the caller pattern, API level)
  c4_lfilter_inf  the same 8 lfilter calls under torch.no_grad (philtorch::lfilter_ss)
  c4_filtfilt  8 x lti.filtfilt(replicate, padlen 9), forward only (philtorch::filtfilt)
  c4_filtfilt_grad  the same plus the gradient w.r.t. x (philtorch::filtfilt_backward)
  c4_filtfilt_coef  the same plus the gradients w.r.t. x, b and a (its coefficient mode)
  c4_lfilter4  4 x lti.lfilter of order 4 (tdf2), forward only (philtorch::lti_ss)
  c4_lfilter4_grad  the same plus gradients w.r.t. x, b and a (philtorch::lfilter_ss_states forward,
                    philtorch::lfilter_ss_backward given its states)
  c4_mimo  lti.state_space of order 4, 2 inputs and 2 outputs per step (philtorch::mimo_ss)
  c4_mimo_grad  the same plus gradients w.r.t. x and zi (the adjoint mimo_ss pass)
  c4_mimo_coef  the same plus gradients w.r.t. A, B, C, D (two states passes and the fused sums)
  c3_lpv_mimo  lpv.state_space on C3's A[t], 2 inputs and 2 outputs per step (philtorch::lpv_mimo_ss)
  c3_lpv_mimo_grad  the same plus gradients w.r.t. x and zi; c3_lpv_mimo_coef: and A[t], B, C, D
--composed runs an API config (c3_lpv_ss*, c3_lpv_mimo*, c4_api, c4_lfilter*, c4_filtfilt*, c4_mimo*)
through the reference's composed route instead of the fused kernels, for the
comparison.
Before every step a 512 MiB buffer is read end to end so the 256 MB Infinity
Cache holds none of the step's operands (a read sweep, not a write: a write
would leave dirty lines whose write-back then competes with the step); the
sweep is outside the timed events.

Output: one JSON line (the driver's contract) with
  value        GSamples/s = samples / t_step, whole job (one GPU); t_step is
               the mean over the K timed steps of one HIP-event pair around
               the step's launches
  roofline     the dominant kernel (the backward scan): algorithmic bytes per
               launch over its mean HIP-event duration from a second pass that
               puts events between the launches, against 8 TB/s; `traffic` is
               the measured HBM bytes per launch from the rocprofv3 --pmc
               summary under profiles/ when one exists for the config
  cpu_baseline the oracle (a C restatement of the reference CPU extension and
               its composite backward, OpenMP over the batch) on a bounded
               sample of the same workload, on this host's cores
--phases adds detail.phases: where a scan launch's time goes, tile by tile
(claim, loads and fold, look-back, pass 2 and stores), from one traced forward
and one traced backward launch (phs_debug_trace_next_launch).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_HBM_GBS = 8000.0
REPO = os.path.dirname(os.path.abspath(__file__))


# ----------------------------------------------------------------------------
# workloads
class Workload:
    """Inputs on the CPU (for the oracle) and on the GPU, plus the step."""

    name = ""
    metric = ""
    dtype_tag = "f32"
    samples = 0
    fwd_bytes = 0  # algorithmic bytes of one forward call (all its launches)
    bwd_bytes = 0  # algorithmic bytes of one backward call
    # algorithmic bytes of the first launch of a call, the one the launch hook
    # times (None: the call is one launch, fwd_bytes / bwd_bytes)
    fwd_launch_bytes = None
    bwd_launch_bytes = None
    kernel = "scan_kernel"  # the library kernel of those launches
    launches = 1  # forward (and backward) calls per step
    # streaming-probe equivalents of one forward / backward launch: (names of
    # the arrays read, names of the arrays written, fp32 elements per array),
    # or None where the launch's traffic is not a set of equal-length arrays.
    # A name the forward writes and the backward reads is one buffer, as in
    # the step (the backward reads the forward's output and coefficients)
    probe_fwd = None
    probe_bwd = None

    def step_fwd(self):
        raise NotImplementedError

    def step_bwd(self, y):
        raise NotImplementedError

    def cpu_step(self, rows, steps, nthreads):
        raise NotImplementedError


class LpvScalar(Workload):
    def __init__(self, name, B, T, dtype):
        import torch

        self.name, self.B, self.T = name, B, T
        self.dtype_tag = "f32" if dtype == "float32" else "f64"
        self.metric = (
            "GSamples/s fwd+bwd and % of HBM peak, 1st-order LPV scan B=64 T=65536 fp32"
            if name == "c1"
            else f"GSamples/s fwd+bwd, 1st-order LPV scan B={B} T={T} {dtype}"
        )
        g = torch.Generator().manual_seed(1 if name == "c1" else 5)
        dt = getattr(torch, dtype)
        if name == "c1":
            a = torch.rand(B, T, generator=g, dtype=torch.float64) * 1.98 - 0.99
        else:  # c5: a = 0.999 tanh(z), z ~ N(0, 2)
            a = 0.999 * torch.tanh(2.0 * torch.randn(B, T, generator=g, dtype=torch.float64))
        x = torch.randn(B, T, generator=g, dtype=torch.float64)
        y0 = torch.randn(B, generator=g, dtype=torch.float64)
        gy = torch.randn(B, T, generator=g, dtype=torch.float64)
        self.cpu = [v.to(dt) for v in (a, x, y0, gy)]
        self.dev = [v.cuda() for v in self.cpu]
        es = 4 if dtype == "float32" else 8
        self.samples = B * T
        self.fwd_bytes = 3 * es * B * T  # read a, x; write y
        self.bwd_bytes = 5 * es * B * T  # read a, g, y; write grad_x, grad_a
        self.probe_fwd = (("a", "x"), ("y",), B * T * es // 4)
        self.probe_bwd = (("a", "y", "g"), ("grad_a", "grad_x"), B * T * es // 4)

    def step_fwd(self):
        import torch

        a, x, y0, _ = self.dev
        return torch.ops.philtorch.recur(a, y0, x)

    def step_bwd(self, y):
        import torch

        a, _, y0, gy = self.dev
        return torch.ops.philtorch.recur_backward(a, y0, y, gy)

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        a, x, y0, gy = (v.numpy()[:rows, ..., :steps] if v.dim() > 1 else v.numpy()[:rows] for v in self.cpu)
        y = oracle.recur(a, y0, x, nthreads=nthreads)
        oracle.recur_bwd(a, y0, y, gy, nthreads=nthreads)


class LtiComplex(Workload):
    """c2: per-channel complex pole p = r e^{i theta}, the diag_state_space call."""

    def __init__(self):
        import torch

        C, T = 1024, 262144
        self.name, self.B, self.T = "c2", C, T
        self.dtype_tag = "c64"
        self.metric = f"GSamples/s fwd+bwd, LTI diagonal scan complex64 C={C} T={T}"
        g = torch.Generator().manual_seed(2)
        r = torch.rand(C, generator=g, dtype=torch.float64) * 0.099 + 0.9
        th = torch.rand(C, generator=g, dtype=torch.float64) * torch.pi
        p = torch.polar(r, th)
        x = torch.complex(torch.randn(C, T, generator=g), torch.randn(C, T, generator=g))
        zi = torch.complex(torch.randn(C, generator=g), torch.randn(C, generator=g))
        gy = torch.complex(torch.randn(C, T, generator=g), torch.randn(C, T, generator=g))
        self.cpu = [p.to(torch.complex64), x, zi, gy]
        self.dev = [v.cuda() for v in self.cpu]
        self.samples = C * T
        self.fwd_bytes = 16 * C * T  # read x, write y (8 B each)
        self.bwd_bytes = 24 * C * T  # read g, y; write grad_x
        self.probe_fwd = (("x",), ("y",), 2 * C * T)
        self.probe_bwd = (("y", "g"), ("grad_x",), 2 * C * T)

    def step_fwd(self):
        import torch

        p, x, zi, _ = self.dev
        return torch.ops.philtorch.lti_recur(p, zi, x)

    def step_bwd(self, y):
        import torch

        p, _, zi, gy = self.dev
        return torch.ops.philtorch.lti_recur_backward(p, zi, y, gy)

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        p, x, zi, gy = (v.numpy() for v in self.cpu)
        y = oracle.lti_recur(p[:rows], zi[:rows], x[:rows, :steps], nthreads=nthreads)
        oracle.lti_recur_bwd(p[:rows], zi[:rows], y, gy[:rows, :steps], nthreads=nthreads)


class LpvBiquad(Workload):
    """c3: per-sample biquad denominators (TDF-II 2x2 companion), smoothed poles."""

    def __init__(self):
        import torch
        import torch.nn.functional as F

        B, T = 32, 1 << 20
        self.name, self.B, self.T = "c3", B, T
        self.metric = f"GSamples/s fwd+bwd, 2nd-order LPV state_space_recursion B={B} T={T} fp32"
        g = torch.Generator().manual_seed(3)
        r = torch.rand(B, T + 63, generator=g, dtype=torch.float64) * 0.48 + 0.5
        th = torch.rand(B, T + 63, generator=g, dtype=torch.float64) * torch.pi
        kern = torch.full((1, 1, 64), 1 / 64, dtype=torch.float64)
        r = F.conv1d(r.unsqueeze(1), kern).squeeze(1)
        th = F.conv1d(th.unsqueeze(1), kern).squeeze(1)
        a1, a2 = -2 * r * torch.cos(th), r * r
        A = torch.zeros(B, T, 2, 2, dtype=torch.float64)
        A[..., 0, 0], A[..., 0, 1], A[..., 1, 0] = -a1, 1.0, -a2
        x = torch.randn(B, T, generator=g, dtype=torch.float64)
        xw = torch.stack([x, torch.zeros_like(x)], -1)
        zi = torch.randn(B, 2, generator=g, dtype=torch.float64)
        gy = torch.randn(B, T, 2, generator=g, dtype=torch.float64)
        self.cpu = [v.float() for v in (A, xw, zi, gy)]
        self.dev = [v.cuda() for v in self.cpu]
        self.samples = B * T
        self.fwd_bytes = 32 * B * T  # read A (16), x (8); write y (8)
        self.bwd_bytes = 56 * B * T  # read A, g, y; write grad_x (8), grad_A (16)

    def step_fwd(self):
        import torch

        A, x, zi, _ = self.dev
        return torch.ops.philtorch.recur2(A, zi, x)

    def step_bwd(self, y):
        import torch

        A, _, zi, gy = self.dev
        return torch.ops.philtorch.recurN_backward(A, zi, y, gy)

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        A, x, zi, gy = (v.numpy() for v in self.cpu)
        y = oracle.recurN(A[:rows, :steps], zi[:rows], x[:rows, :steps], nthreads=nthreads)
        oracle.recurN_bwd(A[:rows, :steps], zi[:rows], y, gy[:rows, :steps], nthreads=nthreads)


class SosCascade(Workload):
    """c4: 8 biquad sections per batch item, each one TDF-II 2x2 LTI scan."""

    def __init__(self):
        import torch

        B, S, T = 16, 8, 480000
        self.name, self.B, self.T, self.S = "c4", B, T, S
        self.metric = f"GSamples/s fwd+bwd, LTI lfilter cascaded SOS x{S} B={B} T={T} fp32 (op level)"
        g = torch.Generator().manual_seed(4)
        r = torch.rand(B, S, generator=g, dtype=torch.float64) * 0.48 + 0.5
        th = torch.rand(B, S, generator=g, dtype=torch.float64) * torch.pi
        a1, a2 = -2 * r * torch.cos(th), r * r
        A = torch.zeros(B, S, 2, 2, dtype=torch.float64)
        A[..., 0, 0], A[..., 0, 1], A[..., 1, 0] = -a1, 1.0, -a2  # companion(a)^T (TDF-II)
        x = torch.randn(B, T, 2, generator=g, dtype=torch.float64)  # B x[t] of the first section
        zi = torch.zeros(B, 2, dtype=torch.float64)
        gy = torch.randn(B, T, 2, generator=g, dtype=torch.float64)
        self.cpu = [v.float() for v in (A, x, zi, gy)]
        self.dev = [v.cuda() for v in self.cpu]
        # each section's coefficients as a tensor of its own, as a cascade
        # holds them (a strided A[:, s] view would add a copy per call)
        self.A_sec = [self.dev[0][:, s].contiguous() for s in range(S)]
        self.samples = B * T  # input samples through the whole cascade
        self.fwd_bytes = 16 * B * T  # per section: read x, write y
        self.bwd_bytes = 24 * B * T  # per section: read g, y; write grad_x
        self.launches = S

    def step_fwd(self):
        import torch

        _, x, zi, _ = self.dev
        ys = []
        for s in range(self.S):
            ys.append(torch.ops.philtorch.lti_recur2(self.A_sec[s], zi, x if s == 0 else ys[-1]))
        return ys

    def step_bwd(self, ys):
        import torch

        _, _, zi, gy = self.dev
        g = gy
        for s in reversed(range(self.S)):
            _, _, g = torch.ops.philtorch.lti_recurN_backward(self.A_sec[s], zi, ys[s], g)
        return g

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        A, x, zi, gy = (v.numpy() for v in self.cpu)
        ys, h = [], x[:rows, :steps]
        for s in range(self.S):
            h = oracle.lti_recurN(A[:rows, s], zi[:rows], h, nthreads=nthreads)
            ys.append(h)
        g = gy[:rows, :steps]
        for s in reversed(range(self.S)):
            _, _, g = oracle.lti_recurN_bwd(A[:rows, s], zi[:rows], ys[s], g, nthreads=nthreads)


class SosFused(Workload):
    """c4_fused: the C4 cascade (16 rows, 8 biquads, T=480000, fp32) through
    the fused cascade op: philtorch::sosfilt + sosfilt_backward, gradients
    w.r.t. x and every section's coefficients (b, a)."""

    def __init__(self):
        import torch

        B, S, T = 16, 8, 480000
        self.name, self.B, self.T, self.S = "c4_fused", B, T, S
        self.metric = f"GSamples/s fwd+bwd, fused SOS cascade x{S} (grad x, b, a) B={B} T={T} fp32"
        g = torch.Generator().manual_seed(4)
        r = torch.rand(B, S, generator=g, dtype=torch.float64) * 0.48 + 0.5
        th = torch.rand(B, S, generator=g, dtype=torch.float64) * torch.pi
        rz = torch.rand(B, S, generator=g, dtype=torch.float64) * 1.2
        thz = torch.rand(B, S, generator=g, dtype=torch.float64) * torch.pi
        one = torch.ones(B, S, dtype=torch.float64)
        sos = torch.stack([one, -2 * rz * torch.cos(thz), rz * rz, one, -2 * r * torch.cos(th), r * r], dim=-1)
        x = torch.randn(B, T, generator=g, dtype=torch.float64)
        gy = torch.randn(B, T, generator=g, dtype=torch.float64)
        self.cpu = [v.float() for v in (sos, x, gy)]
        self.dev = [v.cuda() for v in self.cpu]
        self.samples = B * T
        ck = 16 * B * T // 32  # per section: an fp64 state pair per 32 steps (the backward's lane chunk)
        self.fwd_bytes = 8 * B * T + S * ck  # read x; write y and the state checkpoints
        self.bwd_bytes = 12 * B * T + S * ck  # read x, grad y and the checkpoints; write grad x
        self.launches = 1
        self.kernel = "sos_kernel"

    def step_fwd(self):
        import torch

        sos, x, _ = self.dev
        return torch.ops.philtorch.sosfilt(sos, None, x)

    def step_bwd(self, out):
        import torch

        sos, x, gy = self.dev
        return torch.ops.philtorch.sosfilt_backward(sos, x, out[2], gy, None, True)

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        sos, x, gy = (v.numpy() for v in self.cpu)
        oracle.sosfilt_bwd(sos[:rows], x[:rows, :steps], None, gy[:rows, :steps], nthreads=nthreads)


class SosApi(SosFused):
    """c4_api: the C4 caller pattern through philtorch's API exactly as
    SURVEY's C4 states it, ``for s in range(8): y = lti.lfilter(b[:, s],
    a[:, s], y, form="tdf2", unroll_factor=1)``, then autograd w.r.t. x, b and
    a (every biquad runs the fused kernel on a HIP device)."""

    def __init__(self):
        super().__init__()
        self.name = "c4_api"
        self.metric = f"GSamples/s fwd+bwd, lti.lfilter cascade x{self.S} (grad x, b, a) B={self.B} T={self.T} fp32 (API)"
        self.launches = self.S
        ck = 16 * self.B * self.T // 32  # one section's state checkpoints
        self.fwd_bytes = 8 * self.B * self.T + ck  # per lfilter
        self.bwd_bytes = 12 * self.B * self.T + ck
    def step_fwd(self):
        import torch
        from philtorch_amd import lti

        sos, x, _ = self.dev
        b = sos[..., 0:3].clone().requires_grad_(True)
        a = sos[..., 4:6].clone().requires_grad_(True)
        xr = x.detach().requires_grad_(True)
        y = xr
        for s in range(self.S):
            y = lti.lfilter(b[:, s], a[:, s], y, form="tdf2", unroll_factor=1)
        return y, (xr, b, a)

    def step_bwd(self, out):
        import torch

        y, inputs = out
        return torch.autograd.grad(y, inputs, self.dev[2])


class LfilterInfApi(SosApi):
    """c4_lfilter_inf: the C4 caller pattern's forward at inference, under
    torch.no_grad: ``for s in range(8): y = lti.lfilter(b[:, s], a[:, s], y,
    form="tdf2", unroll_factor=1)`` with b and a columns of the C4 tables.
    Every call runs philtorch::lfilter_ss (B x, the scan, the state shift
    and C h + D x in one pass of the state-space kernel)."""

    def __init__(self):
        super().__init__()
        self.name = "c4_lfilter_inf"
        self.kernel = "ss_kernel"
        self.metric = (f"GSamples/s fwd (no_grad), lti.lfilter cascade x{self.S} (tdf2) B={self.B} T={self.T} "
                       "fp32 (API)")
        self.fwd_bytes = 8 * self.B * self.T  # per lfilter: read x, write y
        self.bwd_bytes = 0

    def step_fwd(self):
        import torch
        from philtorch_amd import lti

        sos, x, _ = self.dev
        b, a = sos[..., 0:3], sos[..., 4:6]
        with torch.no_grad():
            y = x
            for s in range(self.S):
                y = lti.lfilter(b[:, s], a[:, s], y, form="tdf2", unroll_factor=1)
        return y

    def step_bwd(self, out):
        return out

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        sos, x, _ = (v.numpy() for v in self.cpu)
        oracle.sosfilt(sos[:rows], x[:rows, :steps], nthreads=nthreads)


class FiltfiltApi(SosFused):
    """c4_filtfilt: the filtfilt half of the C4 caller pattern, forward only,
    ``for s in range(8): y = lti.filtfilt(b[:, s], a[:, s], y,
    padmode="replicate", padlen=9, unroll_factor=1)`` (each call runs
    philtorch::filtfilt: two state-space passes, the second in reversed
    time, their entry states derived in the kernel)."""

    def __init__(self):
        super().__init__()
        self.name = "c4_filtfilt"
        self.metric = (f"GSamples/s fwd, lti.filtfilt x{self.S} sections (replicate, padlen 9) "
                       f"B={self.B} T={self.T} fp32 (API)")
        self.fwd_bytes = 16 * self.B * self.T  # per filtfilt: two passes, each reads and writes the row
        self.fwd_launch_bytes = 8 * self.B * self.T  # pass 1
        self.bwd_bytes = 0
        self.launches = self.S
        self.kernel = "ss_kernel"
        sos = self.dev[0]
        self.b = [sos[:, s, 0:3].contiguous() for s in range(self.S)]
        self.a = [sos[:, s, 4:6].contiguous() for s in range(self.S)]

    def step_fwd(self):
        from philtorch_amd import lti

        y = self.dev[1]
        for s in range(self.S):
            y = lti.filtfilt(self.b[s], self.a[s], y, padmode="replicate", padlen=9, unroll_factor=1)
        return y

    def step_bwd(self, out):
        return out

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        sos, x, _ = (v.numpy() for v in self.cpu)
        y = x[:rows, :steps]
        for s in range(self.S):
            y = oracle.filtfilt(sos[:rows, s], y, padmode="replicate", padlen=9, nthreads=nthreads)


class FiltfiltGrad(FiltfiltApi):
    """c4_filtfilt_grad: c4_filtfilt with the gradient w.r.t. x
    (torch.autograd.grad against a seeded upstream gradient).  Each
    filtfilt's backward is philtorch::filtfilt_backward: the two passes'
    adjoints, each a state-space launch of the DF-II model in the opposite
    time direction, plus the per-row pad and edge terms."""

    def __init__(self):
        super().__init__()
        self.name = "c4_filtfilt_grad"
        self.metric = (f"GSamples/s fwd+bwd(x), lti.filtfilt x{self.S} sections (replicate, padlen 9) "
                       f"B={self.B} T={self.T} fp32 (API)")
        self.bwd_bytes = 16 * self.B * self.T  # per filtfilt: two adjoint passes, each reads and writes the row
        self.bwd_launch_bytes = 8 * self.B * self.T  # pass 2's adjoint: read g, write dL/dy1

    def step_fwd(self):
        from philtorch_amd import lti

        x = self.dev[1].detach().requires_grad_(True)
        y = x
        for s in range(self.S):
            y = lti.filtfilt(self.b[s], self.a[s], y, padmode="replicate", padlen=9, unroll_factor=1)
        return y, x

    def step_bwd(self, out):
        import torch

        y, x = out
        return torch.autograd.grad(y, x, self.dev[2])

    cpu_step = None  # the oracle restates filtfilt's forward only


class FiltfiltCoefGrad(FiltfiltGrad):
    """c4_filtfilt_coef: c4_filtfilt with the gradients w.r.t. x and every
    section's b and a.  Each filtfilt's forward keeps pass 1's output and
    both passes' states (philtorch::filtfilt_states); its backward is
    philtorch::filtfilt_backward's coefficient mode given them: the two
    adjoint passes with the model's gradient sums, the pads' sums and the
    steady state's in the per-row kernels, the chain rule to b and a."""

    def __init__(self):
        super().__init__()
        self.name = "c4_filtfilt_coef"
        self.metric = (f"GSamples/s fwd+bwd(x, b, a), lti.filtfilt x{self.S} sections (replicate, padlen 9) "
                       f"B={self.B} T={self.T} fp32 (API)")
        # per filtfilt: each forward pass also writes its 2 states (8 B more each); backward: each adjoint
        # reads its input, 2 states and the forward's input, writes its output (20 B)
        self.fwd_bytes += 16 * self.B * self.T
        self.fwd_launch_bytes = 16 * self.B * self.T  # pass 1: read x, write y1 and its states
        self.bwd_bytes = 40 * self.B * self.T
        self.bwd_launch_bytes = 20 * self.B * self.T  # pass 2's adjoint

    def step_fwd(self):
        from philtorch_amd import lti

        x = self.dev[1].detach().requires_grad_(True)
        coefs = [t.detach().requires_grad_(True) for t in self.b + self.a]
        y = x
        for s in range(self.S):
            y = lti.filtfilt(coefs[s], coefs[self.S + s], y, padmode="replicate", padlen=9, unroll_factor=1)
        return y, x, coefs

    def step_bwd(self, out):
        import torch

        y, x, coefs = out
        return torch.autograd.grad(y, [x] + coefs, self.dev[2])


class Lfilter4Api(SosFused):
    """c4_lfilter4: the C4 signal through order-4 filters, forward only: the
    eight C4 biquads of each row multiplied pairwise into four order-4
    filters, ``for s in range(4): y = lti.lfilter(b4[:, s], a4[:, s], y,
    unroll_factor=1)`` (each call runs philtorch::lti_ss: B x, the 4x4 scan,
    the state shift and C h + D x in one pass)."""

    def __init__(self):
        import numpy as np
        import torch

        super().__init__()
        self.name = "c4_lfilter4"
        self.kernel = "ss_kernel"
        self.S4 = self.S // 2
        self.metric = (f"GSamples/s fwd, lti.lfilter order-4 x{self.S4} (tdf2) B={self.B} T={self.T} fp32 (API)")
        sos = self.cpu[0].double()
        self.b4, self.a4 = [], []
        for s in range(self.S4):
            p, q = sos[:, 2 * s], sos[:, 2 * s + 1]
            b4 = torch.stack([torch.tensor(np.polymul(p[r, :3].numpy(), q[r, :3].numpy())) for r in range(self.B)])
            a4 = torch.stack([torch.tensor(np.polymul(p[r, 3:].numpy(), q[r, 3:].numpy())) for r in range(self.B)])
            a4 = a4[:, 1:]
            self.b4.append(b4.float().cuda().contiguous())
            self.a4.append(a4.float().cuda().contiguous())
        self.fwd_bytes = 8 * self.B * self.T  # per lfilter: read x, write y
        self.bwd_bytes = 0
        self.launches = self.S4

    def step_fwd(self):
        from philtorch_amd import lti

        y = self.dev[1]
        for s in range(self.S4):
            y = lti.lfilter(self.b4[s], self.a4[s], y, form="tdf2", unroll_factor=1)
        return y

    def step_bwd(self, out):
        return out

    def cpu_step(self, rows, steps, nthreads):
        import numpy as np

        import oracle

        x = self.cpu[1].numpy()[:rows, :steps]
        for s in range(self.S4):
            b, a = self.b4[s].cpu().numpy()[:rows], self.a4[s].cpu().numpy()[:rows]
            A = np.zeros((rows, 4, 4), dtype=x.dtype)
            A[:, :, 0] = -a
            A[:, np.arange(3), np.arange(1, 4)] = 1.0  # companion(a)^T (TDF-II)
            x, _ = oracle.lti_state_space(A, x, b[:, 1:] - b[:, :1] * a, None, b[:, 0], None, out_idx=0,
                                          nthreads=nthreads)


class LpvSsApi(LpvBiquad):
    """c3_lpv_ss: the C3 signal through a time-varying biquad as
    ``lpv.state_space(A, x, B=b, D=d, zi, unroll_factor=1, out_idx=0)``,
    forward only: A the C3 companion matrices, b[t] = bn[t, 1:] - bn[t, 0] a[t]
    and d[t] = bn[t, 0] for smoothed time-varying zeros (lpv.lfilter's TDF-II
    model; philtorch/lpv/filtering.py:288-333).  Runs philtorch::lpv_ss: B x,
    the scan, the state shift and C h + D x in one pass."""

    def __init__(self):
        import torch
        import torch.nn.functional as F

        super().__init__()
        B, T = self.B, self.T
        self.name = "c3_lpv_ss"
        self.kernel = "lpv_ss_kernel"
        self.metric = f"GSamples/s fwd, LPV biquad lpv.state_space (tdf2, one output) B={B} T={T} fp32 (API)"
        g = torch.Generator().manual_seed(33)
        rz = torch.rand(B, T + 63, generator=g, dtype=torch.float64) * 1.2
        thz = torch.rand(B, T + 63, generator=g, dtype=torch.float64) * torch.pi
        kern = torch.full((1, 1, 64), 1 / 64, dtype=torch.float64)
        rz = F.conv1d(rz.unsqueeze(1), kern).squeeze(1)
        thz = F.conv1d(thz.unsqueeze(1), kern).squeeze(1)
        bn = torch.stack([torch.ones_like(rz), -2 * rz * torch.cos(thz), rz * rz], -1)
        A = self.cpu[0].double()
        a = torch.stack([-A[..., 0, 0], -A[..., 1, 0]], -1)  # (a1, a2) per step
        bv = bn[..., 1:] - bn[..., :1] * a
        d = bn[..., 0]
        x = self.cpu[1][..., 0].double()
        zi = self.cpu[2].double()
        self.cpu = [v.float().contiguous() for v in (A, x, bv, d, zi)]
        self.dev = [v.cuda() for v in self.cpu]
        self.fwd_bytes = 36 * B * T  # read A (16), x, b (8), d; write y
        self.bwd_bytes = 0

    def step_fwd(self):
        from philtorch_amd import lpv

        A, x, bv, d, zi = self.dev
        return lpv.state_space(A, x, B=bv, D=d, zi=zi, unroll_factor=1, out_idx=0)

    def step_bwd(self, out):
        return out

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        A, x, bv, d, zi = (v.numpy() for v in self.cpu)
        oracle.lpv_state_space(A[:rows, :steps], x[:rows, :steps], bv[:rows, :steps], None, d[:rows, :steps],
                               zi[:rows], out_idx=0, nthreads=nthreads)


class LpvSsGrad(LpvSsApi):
    """c3_lpv_ss_grad: c3_lpv_ss plus the gradients w.r.t. x and zi
    (torch.autograd.grad of y against a seeded upstream gradient).  The
    backward is one more philtorch::lpv_ss pass: the adjoint model
    (A[t]^T read in place, input vector e_0, output vector b[t], d[t]) in
    reversed time."""

    def __init__(self):
        import torch

        super().__init__()
        B, T = self.B, self.T
        self.name = "c3_lpv_ss_grad"
        self.metric = (f"GSamples/s fwd+bwd(x, zi), LPV biquad lpv.state_space (tdf2, one output) B={B} T={T} "
                       "fp32 (API)")
        g = torch.Generator().manual_seed(34)
        self.gy_cpu = torch.randn(B, T, generator=g)
        self.gy = self.gy_cpu.cuda()
        self.bwd_bytes = 36 * B * T  # read A (16), b (8), d, g; write grad_x

    def step_fwd(self):
        from philtorch_amd import lpv

        A, x, bv, d, zi = self.dev
        x, zi = x.detach().requires_grad_(True), zi.detach().requires_grad_(True)
        y, _ = lpv.state_space(A, x, B=bv, D=d, zi=zi, unroll_factor=1, out_idx=0)
        return y, x, zi

    def step_bwd(self, out):
        import torch

        y, x, zi = out
        return torch.autograd.grad(y, (x, zi), self.gy)

    def cpu_step(self, rows, steps, nthreads):
        import numpy as np

        import oracle

        A, x, bv, d, zi = (v.numpy() for v in self.cpu)
        A, x, bv, d, zi = A[:rows, :steps], x[:rows, :steps], bv[:rows, :steps], d[:rows, :steps], zi[:rows]
        gy = self.gy_cpu.numpy()[:rows, :steps]
        oracle.lpv_state_space(A, x, bv, None, d, zi, out_idx=0, nthreads=nthreads)
        # the adjoint model over reversed time: state lambda[T - s], input
        # g[T-1-s], A[T-1-s]^T, input vector e_0, output vector b[T-1-s]
        M = A.shape[-1]
        e0 = np.zeros((1, 1, M), dtype=x.dtype)
        e0[..., 0] = 1
        fl = lambda v: np.ascontiguousarray(v[:, ::-1])  # noqa: E731
        oracle.lpv_state_space(fl(np.swapaxes(A, -1, -2)), fl(gy), e0, fl(bv), fl(d), None, nthreads=nthreads)


class Lfilter4Grad(Lfilter4Api):
    """c4_lfilter4_grad: c4_lfilter4 with the gradients w.r.t. x and every
    filter's b and a (torch.autograd.grad against a seeded upstream
    gradient).  Each lfilter's forward keeps its states
    (philtorch::lfilter_ss_states) and its backward is
    philtorch::lfilter_ss_backward given them: the adjoint pass with the
    coefficient sums."""

    def __init__(self):
        import torch

        super().__init__()
        self.name = "c4_lfilter4_grad"
        self.metric = (f"GSamples/s fwd+bwd(x, b, a), lti.lfilter order-4 x{self.S4} (tdf2) B={self.B} T={self.T} "
                       "fp32 (API)")
        g = torch.Generator().manual_seed(44)
        self.gy = torch.randn(self.B, self.T, generator=g).cuda()
        # per lfilter: the forward also writes its 4 states; the adjoint reads g, x, 4 states, writes grad_x
        self.fwd_bytes += 16 * self.B * self.T
        self.bwd_bytes = (4 + 4 + 16 + 4) * self.B * self.T

    def step_fwd(self):
        from philtorch_amd import lti

        x = self.dev[1].detach().requires_grad_(True)
        coefs = [t.detach().requires_grad_(True) for t in self.b4 + self.a4]
        y = x
        for s in range(self.S4):
            y = lti.lfilter(coefs[s], coefs[self.S4 + s], y, form="tdf2", unroll_factor=1)
        return y, x, coefs

    def step_bwd(self, out):
        import torch

        y, x, coefs = out
        return torch.autograd.grad(y, [x] + coefs, self.gy)

    cpu_step = None  # the oracle restates no coefficient gradients of lfilter


class LpvSsCoefGrad(LpvSsGrad):
    """c3_lpv_ss_coef: c3_lpv_ss_grad with the gradients of the time-varying
    A[t], b[t] and d[t] too: the forward keeps its states
    (philtorch::lpv_ss_states), and philtorch::lpv_ss_backward runs the
    adjoint pass writing the per-step coefficient gradients from them."""

    def __init__(self):
        super().__init__()
        B, T = self.B, self.T
        self.name = "c3_lpv_ss_coef"
        self.metric = (f"GSamples/s fwd+bwd(x, zi, A, b, d), LPV biquad lpv.state_space (tdf2, one output) B={B} "
                       f"T={T} fp32 (API)")
        # the forward also writes its 2 states (8); adjoint: read A, b, d, g, x, states (8), write grad_x,
        # grad_A (16), grad_b (8), grad_d
        self.fwd_bytes += 8 * B * T
        self.bwd_bytes = (16 + 8 + 4 + 4 + 4 + 8 + 4 + 16 + 8 + 4) * B * T

    def step_fwd(self):
        from philtorch_amd import lpv

        A, x, bv, d, zi = (t.detach().requires_grad_(True) for t in self.dev)
        y, _ = lpv.state_space(A, x, B=bv, D=d, zi=zi, unroll_factor=1, out_idx=0)
        return y, (A, x, bv, d, zi)

    def step_bwd(self, out):
        import torch

        y, leaves = out
        return torch.autograd.grad(y, leaves, self.gy)

    cpu_step = None  # the oracle restates no coefficient gradients of the LPV state space


class MimoSsApi(Workload):
    """c4_mimo: a two-channel LTI state space on the C4 shape (16 rows of
    480000 steps, fp32): per row an order-4 model (A block-diagonal of the
    TDF-II companion matrices of the row's first two C4 biquads), two inputs
    and two outputs per step, B (4, 2), C (2, 4), D (2, 2) shared by the
    rows, ``lti.state_space(A, x, B, C, D, zi=zi, unroll_factor=1)`` on
    x (16, 480000, 2).  Runs philtorch::mimo_ss: B x, the scan, the state
    shift and C h + D x in one pass; forward only."""

    def __init__(self):
        import torch

        B, T, M, F, P = 16, 480000, 4, 2, 2
        self.name, self.B, self.T, self.M, self.F, self.P = "c4_mimo", B, T, M, F, P
        self.kernel = "mimo_ss_kernel"
        self.metric = (f"GSamples/s fwd, lti.state_space order {M}, {F} inputs, {P} outputs per step "
                       f"B={B} T={T} fp32 (API)")
        g = torch.Generator().manual_seed(45)
        r = torch.rand(B, 2, generator=g, dtype=torch.float64) * 0.48 + 0.5
        th = torch.rand(B, 2, generator=g, dtype=torch.float64) * torch.pi
        A = torch.zeros(B, M, M, dtype=torch.float64)
        for s in range(2):  # companion(1, -2 r cos th, r^2)^T per block
            A[:, 2 * s, 2 * s] = 2 * r[:, s] * torch.cos(th[:, s])
            A[:, 2 * s + 1, 2 * s] = -r[:, s] ** 2
            A[:, 2 * s, 2 * s + 1] = 1.0
        Bm = torch.randn(M, F, generator=g, dtype=torch.float64) / F ** 0.5
        Cm = torch.randn(P, M, generator=g, dtype=torch.float64)
        Dm = torch.randn(P, F, generator=g, dtype=torch.float64)
        x = torch.randn(B, T, F, generator=g, dtype=torch.float64)
        zi = torch.randn(B, M, generator=g, dtype=torch.float64)
        self.cpu = [v.float().contiguous() for v in (A, x, Bm, Cm, Dm, zi)]
        self.dev = [v.cuda() for v in self.cpu]
        self.samples = B * T
        self.fwd_bytes = 4 * (F + P) * B * T  # read x, write y
        self.bwd_bytes = 0

    def step_fwd(self):
        from philtorch_amd import lti

        A, x, Bm, Cm, Dm, zi = self.dev
        return lti.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)

    def step_bwd(self, out):
        return out

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        A, x, Bm, Cm, Dm, zi = (v.numpy() for v in self.cpu)
        oracle.lti_state_space_mimo(A[:rows], x[:rows, :steps], Bm, Cm, Dm, zi[:rows], nthreads=nthreads)


class MimoSsGrad(MimoSsApi):
    """c4_mimo_grad: c4_mimo plus the gradients w.r.t. x and zi
    (torch.autograd.grad against a seeded upstream gradient): one more
    philtorch::mimo_ss pass, the adjoint model (A^T, input matrix C^T,
    output matrix B^T, D^T) in reversed time."""

    def __init__(self):
        import torch

        super().__init__()
        B, T, F, P = self.B, self.T, self.F, self.P
        self.name = "c4_mimo_grad"
        self.metric = (f"GSamples/s fwd+bwd(x, zi), lti.state_space order {self.M}, {F} inputs, {P} outputs per step "
                       f"B={B} T={T} fp32 (API)")
        g = torch.Generator().manual_seed(46)
        self.gy_cpu = torch.randn(B, T, P, generator=g)
        self.gy = self.gy_cpu.cuda()
        self.bwd_bytes = 4 * (P + F) * B * T  # read g, write grad_x

    def step_fwd(self):
        from philtorch_amd import lti

        A, x, Bm, Cm, Dm, zi = self.dev
        x, zi = x.detach().requires_grad_(True), zi.detach().requires_grad_(True)
        y, _ = lti.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)
        return y, x, zi

    def step_bwd(self, out):
        import torch

        y, x, zi = out
        return torch.autograd.grad(y, (x, zi), self.gy)

    def cpu_step(self, rows, steps, nthreads):
        import numpy as np

        import oracle

        A, x, Bm, Cm, Dm, zi = (v.numpy() for v in self.cpu)
        A, x, zi = A[:rows], x[:rows, :steps], zi[:rows]
        gy = self.gy_cpu.numpy()[:rows, :steps]
        oracle.lti_state_space_mimo(A, x, Bm, Cm, Dm, zi, nthreads=nthreads)
        # the adjoint model over reversed time
        fl = lambda v: np.ascontiguousarray(v[:, ::-1])  # noqa: E731
        oracle.lti_state_space_mimo(np.ascontiguousarray(np.swapaxes(A, -1, -2)), fl(gy), Cm.T.copy(), Bm.T.copy(),
                                    Dm.T.copy(), None, nthreads=nthreads)


class MimoSsCoefGrad(MimoSsGrad):
    """c4_mimo_coef: c4_mimo_grad with the gradients of A, B, C and D too:
    the forward again writing its states (C = I), the adjoint writing its
    states (which also gives grad_zi), and one philtorch::mimo_ss_grad_sums
    pass that sums the four products over time (and rows, for the shared B,
    C, D) and writes grad_x = B^T lambda + D^T g."""

    def __init__(self):
        super().__init__()
        B, T, M, F, P = self.B, self.T, self.M, self.F, self.P
        self.name = "c4_mimo_coef"
        self.metric = (f"GSamples/s fwd+bwd(x, zi, A, B, C, D), lti.state_space order {M}, {F} inputs, {P} outputs "
                       f"per step B={B} T={T} fp32 (API)")
        # states (read x, write h), adjoint states (read g, write lambda), then the sums pass (read
        # lambda, h, x, g; write grad_x)
        self.bwd_bytes = 4 * ((F + M) + (P + M) + (M + M + F + P + F)) * B * T
        self.bwd_launch_bytes = 4 * (F + M) * B * T  # the states pass

    def step_fwd(self):
        from philtorch_amd import lti

        leaves = [t.detach().requires_grad_(True) for t in self.dev]
        A, x, Bm, Cm, Dm, zi = leaves
        y, _ = lti.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)
        return y, leaves

    def step_bwd(self, out):
        import torch

        y, leaves = out
        return torch.autograd.grad(y, leaves, self.gy)

    cpu_step = None  # the oracle restates no coefficient gradients of the state space


class LpvMimoApi(LpvBiquad):
    """c3_lpv_mimo: the C3 time-varying biquad dynamics A[t] (32 rows of 2^20
    steps, fp32) with two inputs and two outputs per step, B (2, 2), C (2, 2),
    D (2, 2) shared by the rows: ``lpv.state_space(A, x, B, C, D, zi=zi,
    unroll_factor=1)`` on x (32, 2^20, 2).  Runs philtorch::lpv_mimo_ss: B x,
    the scan, the state shift and C h + D x in one pass; forward only."""

    def __init__(self):
        import torch

        super().__init__()
        B, T = self.B, self.T
        self.name = "c3_lpv_mimo"
        self.kernel = "lpv_mimo_kernel"
        self.metric = f"GSamples/s fwd, LPV lpv.state_space order 2, 2 inputs, 2 outputs per step B={B} T={T} fp32 (API)"
        g = torch.Generator().manual_seed(35)
        A = self.cpu[0]
        x = torch.randn(B, T, 2, generator=g)
        Bm = torch.randn(2, 2, generator=g) / 2 ** 0.5
        Cm, Dm = torch.randn(2, 2, generator=g), torch.randn(2, 2, generator=g)
        zi = torch.randn(B, 2, generator=g)
        self.cpu = [v.contiguous() for v in (A, x, Bm, Cm, Dm, zi)]
        self.dev = [v.cuda() for v in self.cpu]
        self.fwd_bytes = 32 * B * T  # read A (16), x (8); write y (8)
        self.bwd_bytes = 0

    def step_fwd(self):
        from philtorch_amd import lpv

        A, x, Bm, Cm, Dm, zi = self.dev
        return lpv.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)

    def step_bwd(self, out):
        return out

    def cpu_step(self, rows, steps, nthreads):
        import oracle

        A, x, Bm, Cm, Dm, zi = (v.numpy() for v in self.cpu)
        oracle.lpv_state_space_mimo(A[:rows, :steps], x[:rows, :steps], Bm, Cm, Dm, zi[:rows], nthreads=nthreads)


class LpvMimoGrad(LpvMimoApi):
    """c3_lpv_mimo_grad: c3_lpv_mimo plus the gradients w.r.t. x and zi: one
    more philtorch::lpv_mimo_ss pass, the adjoint model (A[t]^T read in
    place, input matrix C^T, output matrix B^T, D^T) in reversed time."""

    def __init__(self):
        import torch

        super().__init__()
        B, T = self.B, self.T
        self.name = "c3_lpv_mimo_grad"
        self.metric = (f"GSamples/s fwd+bwd(x, zi), LPV lpv.state_space order 2, 2 inputs, 2 outputs per step "
                       f"B={B} T={T} fp32 (API)")
        g = torch.Generator().manual_seed(36)
        self.gy_cpu = torch.randn(B, T, 2, generator=g)
        self.gy = self.gy_cpu.cuda()
        self.bwd_bytes = 32 * B * T  # read A (16), g (8); write grad_x (8)

    def step_fwd(self):
        from philtorch_amd import lpv

        A, x, Bm, Cm, Dm, zi = self.dev
        x, zi = x.detach().requires_grad_(True), zi.detach().requires_grad_(True)
        y, _ = lpv.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)
        return y, x, zi

    def step_bwd(self, out):
        import torch

        y, x, zi = out
        return torch.autograd.grad(y, (x, zi), self.gy)

    def cpu_step(self, rows, steps, nthreads):
        import numpy as np

        import oracle

        A, x, Bm, Cm, Dm, zi = (v.numpy() for v in self.cpu)
        A, x, zi = A[:rows, :steps], x[:rows, :steps], zi[:rows]
        gy = self.gy_cpu.numpy()[:rows, :steps]
        oracle.lpv_state_space_mimo(A, x, Bm, Cm, Dm, zi, nthreads=nthreads)
        fl = lambda v: np.ascontiguousarray(v[:, ::-1])  # noqa: E731
        oracle.lpv_state_space_mimo(fl(np.swapaxes(A, -1, -2)), fl(gy), Cm.T.copy(), Bm.T.copy(), Dm.T.copy(), None,
                                    nthreads=nthreads)


class LpvMimoCoefGrad(LpvMimoGrad):
    """c3_lpv_mimo_coef: c3_lpv_mimo_grad with the gradients of A[t], B, C and
    D too: the forward keeps its states (philtorch::lpv_mimo_ss_states), the
    adjoint writes its states (which also gives grad_zi), and one
    philtorch::mimo_ss_grad_sums pass writes dL/dA[t] = lambda[t+1] h[t]^T
    and grad_x = B^T lambda + D^T g per step and sums over time for B, C,
    D."""

    def __init__(self):
        super().__init__()
        B, T = self.B, self.T
        self.name = "c3_lpv_mimo_coef"
        self.metric = (f"GSamples/s fwd+bwd(x, zi, A, B, C, D), LPV lpv.state_space order 2, 2 inputs, 2 outputs "
                       f"per step B={B} T={T} fp32 (API)")
        # the forward also writes its 2 states (8); backward: the adjoint-states pass (32: A, g in,
        # lambda out) and the sums pass (read lambda, h, x, g: 32; write dL/dA[t]: 16, grad_x: 8)
        self.fwd_bytes += 8 * B * T
        self.bwd_bytes = (32 + 56) * B * T
        self.bwd_launch_bytes = 32 * B * T  # the adjoint-states pass

    def step_fwd(self):
        from philtorch_amd import lpv

        leaves = [t.detach().requires_grad_(True) for t in self.dev]
        A, x, Bm, Cm, Dm, zi = leaves
        y, _ = lpv.state_space(A, x, Bm, Cm, Dm, zi=zi, unroll_factor=1)
        return y, leaves

    def step_bwd(self, out):
        import torch

        y, leaves = out
        return torch.autograd.grad(y, leaves, self.gy)

    cpu_step = None  # the oracle restates no coefficient gradients of the state space


def make_workload(name):
    if name == "c1":
        return LpvScalar("c1", 64, 65536, "float32")
    if name == "c5":
        return LpvScalar("c5", 8, 1 << 24, "float32")
    if name == "c5_f64":
        return LpvScalar("c5_f64", 8, 1 << 24, "float64")
    if name == "c2":
        return LtiComplex()
    if name == "c3":
        return LpvBiquad()
    if name == "c4":
        return SosCascade()
    if name == "c4_fused":
        return SosFused()
    if name == "c4_api":
        return SosApi()
    if name == "c4_filtfilt":
        return FiltfiltApi()
    if name == "c4_filtfilt_grad":
        return FiltfiltGrad()
    if name == "c4_filtfilt_coef":
        return FiltfiltCoefGrad()
    if name == "c4_lfilter_inf":
        return LfilterInfApi()
    if name == "c4_lfilter4":
        return Lfilter4Api()
    if name == "c3_lpv_ss":
        return LpvSsApi()
    if name == "c3_lpv_ss_grad":
        return LpvSsGrad()
    if name == "c3_lpv_ss_coef":
        return LpvSsCoefGrad()
    if name == "c4_lfilter4_grad":
        return Lfilter4Grad()
    if name == "c4_mimo":
        return MimoSsApi()
    if name == "c4_mimo_grad":
        return MimoSsGrad()
    if name == "c4_mimo_coef":
        return MimoSsCoefGrad()
    if name == "c3_lpv_mimo":
        return LpvMimoApi()
    if name == "c3_lpv_mimo_grad":
        return LpvMimoGrad()
    if name == "c3_lpv_mimo_coef":
        return LpvMimoCoefGrad()
    raise ValueError(name)


API_CONFIGS = ("c3_lpv_ss", "c3_lpv_ss_grad", "c3_lpv_ss_coef", "c4_api", "c4_lfilter_inf", "c4_filtfilt",
               "c4_filtfilt_grad", "c4_filtfilt_coef", "c4_lfilter4", "c4_lfilter4_grad", "c4_mimo", "c4_mimo_grad",
               "c4_mimo_coef", "c3_lpv_mimo", "c3_lpv_mimo_grad", "c3_lpv_mimo_coef")
CONFIGS = ("c1", "c2", "c3", "c3_lpv_ss", "c3_lpv_ss_grad", "c3_lpv_ss_coef", "c4", "c4_fused", "c4_api",
           "c4_lfilter_inf", "c4_filtfilt", "c4_filtfilt_grad", "c4_filtfilt_coef", "c4_lfilter4", "c4_lfilter4_grad",
           "c4_mimo", "c4_mimo_grad", "c4_mimo_coef", "c3_lpv_mimo", "c3_lpv_mimo_grad", "c3_lpv_mimo_coef", "c5",
           "c5_f64")


# ----------------------------------------------------------------------------
def cpu_model() -> str:
    """The host CPU's model name (first `model name` line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w: Workload, budget_s=10.0):
    """Time the oracle's forward + backward on a bounded sample of rows
    (None where the oracle has no restatement of the config's backward)."""
    import statistics

    if w.cpu_step is None:
        return None
    cores = len(os.sched_getaffinity(0))
    rows = min(w.B, max(cores, 1))  # the reference parallelises over rows only
    # bound one repetition: all sampled rows over a prefix of the time axis
    steps = int(min(w.T, 64e6 // (rows * w.launches)))
    t0 = time.perf_counter()
    w.cpu_step(rows, steps, cores)
    probe = time.perf_counter() - t0
    reps = int(max(1, min(50, budget_s / max(probe, 1e-6))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        w.cpu_step(rows, steps, cores)
        times.append(time.perf_counter() - t0)
    med = float(statistics.median(times))
    return {
        "value": rows * steps / med / 1e9,
        "unit": "GSamples/s",
        "cores": cores,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"{rows} of {w.B} rows x the first {steps} of T={w.T} steps, {'fwd+bwd' if w.bwd_bytes else 'fwd'}, median of {reps} reps "
        f"(oracle/phs_oracle.c, OpenMP over rows, {cores} threads)",
    }


def _measured_traffic(config, direction="backward"):
    """HBM bytes of one launch of the dominant kernel (the first launch of a
    call, the one the launch hook times), from the rocprofv3 --pmc summary
    committed under profiles/ (FETCH_SIZE + WRITE_SIZE, each scaled by the
    same counter on a plain copy of known size), or None."""
    path = os.path.join(REPO, "profiles", f"traffic_{config}.json")
    key = "bwd_bytes_per_launch" if direction == "backward" else "fwd_bytes_per_launch"
    try:
        with open(path) as f:
            return json.load(f)[key]
    except (OSError, KeyError, ValueError):
        return None


def _kernel_lib():
    """libphilscan through ctypes (the process's already loaded copy) for its
    measurement hook and streaming probe."""
    import ctypes

    import philtorch_amd

    lib = ctypes.CDLL(philtorch_amd.KERNEL_LIBRARY)
    lib.phs_debug_time_next_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.phs_debug_time_next_launch.restype = None
    lib.phs_stream_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p]
    lib.phs_stream_probe.restype = ctypes.c_int
    lib.phs_debug_trace_next_launch.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.phs_debug_trace_next_launch.restype = None
    return lib


def _fresh_events():
    """Two timing events, created (recorded once) so that their handles exist
    before the launch hook records them around a kernel."""
    import torch

    ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    for e in ev:
        e.record()
    return ev


def _ceiling(lib, w, steps, evict_caches, dev):
    """The streaming probe (phs_stream_probe) moving one step's bytes: the
    forward launch's arrays, then the backward's over the same buffers the
    step uses (the backward re-reads the forward's coefficients and output),
    with the same cache eviction before every step.  Reports the step time, each kernel's own
    duration (launch hook) and the scan step's fraction of it; the tile shape
    of the scalar scan (shape 0) and a flat one-vector-per-lane shape (shape
    1) are both timed and the faster is reported.  None where the workload's
    launches are not equal-length array streams."""
    import ctypes

    import torch

    if w.probe_fwd is None or w.probe_bwd is None:
        return None
    if any(p[2] % 8192 for p in (w.probe_fwd, w.probe_bwd)):
        return None
    bufs = {}

    def arrays(ins_named, outs_named, n):
        for nm in ins_named + outs_named:
            if nm not in bufs:
                bufs[nm] = torch.ones(n, dtype=torch.float32, device=dev)
        ins = (ctypes.c_void_p * 3)(*[bufs[nm].data_ptr() for nm in ins_named])
        outs = (ctypes.c_void_p * 2)(*[bufs[nm].data_ptr() for nm in outs_named])
        return ins, outs

    calls = [((len(p[0]), len(p[1]), p[2]), arrays(*p)) for p in (w.probe_fwd, w.probe_bwd)]
    results = {}
    for shape in (0, 1):
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

        def probe_step(timed=None):
            for j, ((n_in, n_out, n), (ins, outs)) in enumerate(calls):
                if timed is not None:
                    lib.phs_debug_time_next_launch(timed[j][0].cuda_event, timed[j][1].cuda_event)
                rc = lib.phs_stream_probe(shape, n_in, n_out, n, ins, outs, stream)
                if rc != 0:
                    raise RuntimeError(f"phs_stream_probe returned {rc}")

        for _ in range(3):
            evict_caches()
            probe_step()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i in range(steps):
            evict_caches()
            ev[i][0].record()
            probe_step()
            ev[i][1].record()
        kev = []
        for i in range(steps):
            evict_caches()
            k = [_fresh_events(), _fresh_events()]
            probe_step(k)
            kev.append(k)
        lib.phs_debug_time_next_launch(None, None)
        torch.cuda.synchronize()
        results[shape] = (
            sum(a.elapsed_time(b) for a, b in ev) / steps,
            sum(k[0][0].elapsed_time(k[0][1]) for k in kev) / steps,
            sum(k[1][0].elapsed_time(k[1][1]) for k in kev) / steps,
        )
    best = min(results, key=lambda sh: results[sh][0])
    ms_step, ms_f, ms_b = results[best]
    step_bytes = (w.fwd_bytes + w.bwd_bytes) * w.launches
    del bufs, calls
    # a plain device copy (torch's copy_, the runtime's own copy kernel)
    # moving the same bytes as each launch: half of them read, half written
    copies = {}
    for nm, nbytes in (("fwd", w.fwd_bytes), ("bwd", w.bwd_bytes)):
        src = torch.ones(nbytes // 8, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            evict_caches()
            dst.copy_(src)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i in range(steps):
            evict_caches()
            ev[i][0].record()
            dst.copy_(src)
            ev[i][1].record()
        torch.cuda.synchronize()
        copies[nm] = sum(a.elapsed_time(b) for a, b in ev) / steps
        del src, dst
    return {
        "kernel": f"phs_stream_probe shape {best} ({'scan tile geometry' if best == 0 else 'one float4 per lane'})",
        "ms_per_step": round(ms_step, 5),
        "ms_fwd_kernel": round(ms_f, 5),
        "ms_bwd_kernel": round(ms_b, 5),
        "step_GBs": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        "step_frac_of_peak": round(step_bytes / (ms_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "shapes_ms_per_step": {str(k): round(v[0], 5) for k, v in results.items()},
        "device_copy": {
            "what": "torch copy_ of a buffer of half each launch's bytes (reads + writes = the launch's bytes), "
                    "one event pair around each copy, same cache eviction",
            "ms_fwd_equivalent": round(copies["fwd"], 5),
            "ms_bwd_equivalent": round(copies["bwd"], 5),
            "GBs_fwd_equivalent": round(w.fwd_bytes / (copies["fwd"] * 1e-3) / 1e9, 1),
            "GBs_bwd_equivalent": round(w.bwd_bytes / (copies["bwd"] * 1e-3) / 1e9, 1),
        },
    }


def _phases(lib, w, evict_caches, dev):
    """Per-tile phase breakdown of the first forward and the first backward
    scan launch of a step, from the tracing build of the scan kernel
    (phs_debug_trace_next_launch): per tile, the tile claim, data wave 0's
    loads and fold, the wait for the other waves' aggregates, the look-back
    (entry state known) and pass 2 with its stores; percentiles in us over
    the launch's tiles, and the failed look-back polls.  None for workloads
    whose kernel is not scan_kernel."""
    import numpy as np
    import torch

    if w.kernel != "scan_kernel":
        return None
    n = 1 << 18
    rec = torch.zeros(n * 8, dtype=torch.int64, device=dev)
    out = {}
    for direction in ("forward", "backward"):
        evict_caches()
        rec.zero_()
        torch.cuda.synchronize()
        if direction == "forward":
            lib.phs_debug_trace_next_launch(rec.data_ptr(), n)
            w.step_fwd()
        else:
            y = w.step_fwd()
            lib.phs_debug_trace_next_launch(rec.data_ptr(), n)
            w.step_bwd(y)
        torch.cuda.synchronize()
        lib.phs_debug_trace_next_launch(None, 0)
        r = rec.view(-1, 8).cpu().numpy()
        r = r[r[:, 0] != 0].astype(np.float64)
        if len(r) == 0:
            out[direction] = None
            continue
        start, claimed, loaded, aggs, entry, stored = (r[:, i] * 0.01 for i in range(6))  # 100 MHz -> us
        pct = lambda v: [round(float(np.percentile(v, p)), 2) for p in (10, 50, 90)]  # noqa: E731
        out[direction] = {
            "tiles": int(len(r)),
            "percentiles": [10, 50, 90],
            "claim_us": pct(claimed - start),
            "load_fold_us": pct(loaded - claimed),
            "wait_aggregates_us": pct(aggs - loaded),
            "lookback_us": pct(entry - aggs),
            "pass2_store_us": pct(stored - entry),
            "tile_life_us": pct(stored - start),
            "start_spread_us": round(float(start.max() - start.min()), 2),
            "wave_span_us": round(float(stored.max() - start.min()), 2),
            "failed_polls": [int(np.percentile(r[:, 6], p)) for p in (10, 50, 90)],
        }
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c1", choices=CONFIGS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--phases", action="store_true",
                    help="add the per-tile phase breakdown of a traced forward and backward scan launch")
    ap.add_argument("--no-evict", action="store_true", help="keep operands cache-resident (diagnostic)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="after timing, run one plain 256 MiB device copy (reads and writes 256 MiB) so "
                    "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE of this run can be scaled to bytes")
    ap.add_argument("--composed", action="store_true",
                    help=f"run an API config ({', '.join(API_CONFIGS)}) through the reference's composed route "
                    "(the fused state-space, lfilter, biquad and filtfilt routes switched off), for comparison")
    args = ap.parse_args()
    if args.composed and args.config not in API_CONFIGS:
        ap.error(f"--composed applies to {', '.join(API_CONFIGS)}")

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: the linear-recurrence path shards over batch rows "
            "with no communication, and this build runs and reports a single MI355X.",
            file=sys.stderr,
        )
        return 2

    import torch

    sys.path.insert(0, REPO)
    import philtorch_amd

    philtorch_amd.require_extension()
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2

    w = make_workload(args.config)
    if args.composed:
        from philtorch_amd.lpv import ssm as lpv_ssm
        from philtorch_amd.lti import filtering, ssm as lti_ssm

        off = lambda *a, **k: False  # noqa: E731
        for mod, fn in ((lpv_ssm, "_fused_lpv_ss_applies"), (lpv_ssm, "_lpv_mimo_applies"),
                        (lti_ssm, "_fused_ss_applies"), (lti_ssm, "_mimo_applies"), (filtering, "_fused_biquad_applies"),
                        (filtering, "_fused_lfilter_applies"), (filtering, "_fused_filtfilt_applies")):
            setattr(mod, fn, off)
        w.metric += " [composed route]"
    dev = torch.device("cuda", 0)
    evict = None if args.no_evict else torch.ones(128 << 20, dtype=torch.float32, device=dev)
    evict_sink = torch.empty((), dtype=torch.float32, device=dev)

    def evict_caches():
        if evict is not None:
            torch.sum(evict, dim=0, out=evict_sink)

    for _ in range(args.warmup):
        evict_caches()
        w.step_bwd(w.step_fwd())
    torch.cuda.synchronize()

    # timed region: K steps, each bracketed by one event pair (the cache
    # eviction before each step stays outside the events)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for i in range(args.steps):
        evict_caches()
        ev[i][0].record()
        w.step_bwd(w.step_fwd())
        ev[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps

    # kernel pass: the same steps, each forward and backward main kernel
    # timed by the library's launch hook (events recorded around the kernel
    # itself, as rocprofv3's kernel trace measures it), first launch of each
    # direction per step
    lib = _kernel_lib()
    kev = []
    for i in range(args.steps):
        evict_caches()
        fe, be = _fresh_events(), _fresh_events()
        lib.phs_debug_time_next_launch(fe[0].cuda_event, fe[1].cuda_event)
        y = w.step_fwd()
        if w.bwd_bytes:
            lib.phs_debug_time_next_launch(be[0].cuda_event, be[1].cuda_event)
        w.step_bwd(y)
        kev.append((fe, be))
    lib.phs_debug_time_next_launch(None, None)
    torch.cuda.synchronize()
    mean_fwd = sum(f[0].elapsed_time(f[1]) for f, _ in kev) / args.steps
    mean_bwd = sum(b[0].elapsed_time(b[1]) for _, b in kev) / args.steps if w.bwd_bytes else 0.0
    fwd_lb = w.fwd_launch_bytes or w.fwd_bytes
    bwd_lb = w.bwd_launch_bytes or w.bwd_bytes
    if w.bwd_bytes and mean_bwd >= mean_fwd:
        dominant = ("backward", bwd_lb, mean_bwd)
    else:
        dominant = ("forward", fwd_lb, mean_fwd)
    achieved = dominant[1] / (dominant[2] * 1e-3) / 1e9
    step_bytes = (w.fwd_bytes + w.bwd_bytes) * w.launches
    ceiling = _ceiling(lib, w, args.steps, evict_caches, dev)

    result = {
        "metric": w.metric,
        "value": round(w.samples / (ms_per_step * 1e-3) / 1e9, 3),
        "unit": "GSamples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype_tag,
        "data": "synthetic (seeded torch.Generator, CPU-generated, copied to HBM before timing)",
        "config": {
            "workload": {
                "c1": "lpv_scan_fwd_bwd_B64_T65536_f32",
                "c2": "lti_diag_scan_fwd_bwd_C1024_T262144_c64",
                "c3": "lpv_2x2_scan_fwd_bwd_B32_T1048576_f32",
                "c4": "lti_sos8_cascade_fwd_bwd_B16_T480000_f32",
                "c4_fused": "lti_sos8_cascade_fused_fwd_bwd_B16_T480000_f32",
                "c4_api": "lti_lfilter8_cascade_api_fwd_bwd_B16_T480000_f32",
                "c4_filtfilt": "lti_filtfilt8_api_fwd_B16_T480000_f32",
                "c4_filtfilt_grad": "lti_filtfilt8_api_fwd_bwd_x_B16_T480000_f32",
                "c4_filtfilt_coef": "lti_filtfilt8_api_fwd_bwd_x_b_a_B16_T480000_f32",
                "c4_lfilter_inf": "lti_lfilter8_cascade_api_fwd_nograd_B16_T480000_f32",
                "c4_lfilter4": "lti_lfilter_order4_x4_api_fwd_B16_T480000_f32",
                "c3_lpv_ss": "lpv_biquad_state_space_api_fwd_B32_T1048576_f32",
                "c3_lpv_ss_grad": "lpv_biquad_state_space_api_fwd_bwd_x_zi_B32_T1048576_f32",
                "c3_lpv_ss_coef": "lpv_biquad_state_space_api_fwd_bwd_all_B32_T1048576_f32",
                "c4_lfilter4_grad": "lti_lfilter_order4_x4_api_fwd_bwd_x_b_a_B16_T480000_f32",
                "c4_mimo": "lti_state_space_order4_2in_2out_api_fwd_B16_T480000_f32",
                "c4_mimo_grad": "lti_state_space_order4_2in_2out_api_fwd_bwd_x_zi_B16_T480000_f32",
                "c4_mimo_coef": "lti_state_space_order4_2in_2out_api_fwd_bwd_all_B16_T480000_f32",
                "c3_lpv_mimo": "lpv_state_space_order2_2in_2out_api_fwd_B32_T1048576_f32",
                "c3_lpv_mimo_grad": "lpv_state_space_order2_2in_2out_api_fwd_bwd_x_zi_B32_T1048576_f32",
                "c3_lpv_mimo_coef": "lpv_state_space_order2_2in_2out_api_fwd_bwd_all_B32_T1048576_f32",
                "c5": "lpv_scan_fwd_bwd_B8_T16777216_f32",
                "c5_f64": "lpv_scan_fwd_bwd_B8_T16777216_f64",
            }[w.name],
            "B": w.B,
            "T": w.T,
            "cache_evicted_between_steps": evict is not None,
        },
        "detail": {
            "route": "composed" if args.composed else "fused",
            "launches_per_direction": w.launches,
            "ms_fwd_kernel": round(mean_fwd, 5),
            "ms_bwd_kernel": round(mean_bwd, 5) if w.bwd_bytes else None,
            "kernel_timing": "library launch hook: events recorded around the kernel by hipExtLaunchKernelGGL",
            "fwd_launch_bytes": fwd_lb,
            "bwd_launch_bytes": bwd_lb if w.bwd_bytes else None,
            "fwd_GBs_algorithmic": round(fwd_lb / (mean_fwd * 1e-3) / 1e9, 1),
            "bwd_GBs_algorithmic": round(bwd_lb / (mean_bwd * 1e-3) / 1e9, 1) if w.bwd_bytes else None,
            "fwd_frac": round(fwd_lb / (mean_fwd * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "bwd_frac": round(bwd_lb / (mean_bwd * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if w.bwd_bytes else None,
            "wall_s_timed_region": round(wall, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{w.kernel} ({dominant[0]}, first launch of a call)",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": None if args.composed else _measured_traffic(w.name, dominant[0]),
            "step_GBs_algorithmic": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
            "step_frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "ceiling": ceiling,
        },
    }
    if ceiling is not None:
        ceiling["scan_step_frac_of_ceiling"] = round(ceiling["ms_per_step"] / ms_per_step, 4)
    if args.phases:
        result["detail"]["phases"] = _phases(lib, w, evict_caches, dev)
    if args.calib_copy:
        csrc = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        cdst = torch.empty_like(csrc)
        torch.cuda.synchronize()
        evict_caches()
        cdst.copy_(csrc)
        torch.cuda.synchronize()
        result["detail"]["calib_copy_bytes_each_way"] = 256 << 20
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
