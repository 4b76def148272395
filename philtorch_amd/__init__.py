"""philtorch_amd — MI355X-native linear-recurrence core with philtorch's API.

Importing the package loads ``_C.so`` (the torch.library layer over the HIP
kernels of ``libphilscan.so``), which defines the ``philtorch`` operator
namespace: the reference's five ops (``recur2``, ``recurN``, ``lti_recur2``,
``lti_recurN``, ``lti_recur``; philtorch/csrc/host_recur2.cpp:162-171), the new
LPV scalar op ``recur``, four fused backward ops, and the fused cascade of
second-order sections ``sosfilt`` / ``sosfilt_backward`` (no reference
counterpart; ``lti.sosfilt`` is its API), the forward-only zero-phase
``filtfilt`` of filters up to order 4 (behind ``lti.filtfilt``) and the
fused single-input single-output state space ``lti_ss`` (behind
``lti.state_space``), ``lfilter_ss``, ``lfilter`` of order <= 4 from b and
a in one pass (behind ``lti.lfilter``), ``lpv_ss``, the time-varying
single-input single-output state space of order <= 4 (behind
``lpv.state_space``), ``mimo_ss``, the LTI state space of order <= 4
with up to four inputs and outputs per step (behind ``lti.state_space``
for a 3D x or matrix-valued B, C, D), and ``lpv_mimo_ss``, its LPV form
(behind ``lpv.state_space``).  This module then
registers fake (meta) kernels and autograd formulas for them, as
philtorch/__init__.py:157-268 does for its ops.

Backward: without ``create_graph`` the registered formula calls the fused
single-pass adjoint kernel (``*_backward`` ops).  With ``create_graph`` it
falls back to the composite formula written with the same ops, which is
differentiable again (gradgradcheck).

If the extension is missing, ``EXTENSION_LOADED`` is False and the Python API
takes philtorch's pure-PyTorch route, as the reference does
(philtorch/__init__.py:6-12); on a machine with a GPU the import fails instead,
so a GPU run can never silently lose its kernels
(set PHILTORCH_AMD_ALLOW_MISSING_EXTENSION=1 to override).
"""
from __future__ import annotations

import os
import warnings
from typing import Any, Optional

import torch

__version__ = "0.1.0"

_HERE = os.path.dirname(os.path.abspath(__file__))
OPS_LIBRARY = os.path.join(_HERE, "_C.so")
KERNEL_LIBRARY = os.path.join(_HERE, "libphilscan.so")


def _load_extension() -> tuple[bool, Optional[BaseException]]:
    if not os.path.exists(OPS_LIBRARY):
        return False, FileNotFoundError(OPS_LIBRARY)
    try:
        torch.ops.load_library(OPS_LIBRARY)
    except (OSError, RuntimeError) as exc:  # pragma: no cover - depends on the build
        return False, exc
    return True, None


EXTENSION_LOADED, _LOAD_ERROR = _load_extension()
HELION_LOADED = False  # the Helion backend of the reference is out of scope

if not EXTENSION_LOADED:
    if torch.cuda.is_available() and not os.environ.get("PHILTORCH_AMD_ALLOW_MISSING_EXTENSION"):
        raise ImportError(
            f"philtorch_amd: the HIP extension {OPS_LIBRARY} did not load ({_LOAD_ERROR}); "
            "build it with `python -m philtorch_amd._build`"
        )
    warnings.warn("Custom extension not loaded.")


def require_extension() -> None:
    """Raise unless the native operators are available."""
    if not EXTENSION_LOADED:
        raise RuntimeError(
            f"philtorch_amd native extension not loaded ({_LOAD_ERROR}); "
            "build it with `python -m philtorch_amd._build`"
        )


# --------------------------------------------------------------------------
# composite backward formulas (used when create_graph=True)
#
# Adjoint of h[t] = A[t] h[t-1] + x[t]:
#   lambda[t] = g[t] + A[t+1]^H lambda[t+1],  lambda[T-1] = g[T-1]
#   grad_x = lambda,  grad_zi = A[0]^H lambda[0],  grad_A[t] = lambda[t] conj(h[t-1])^T
# (philtorch/__init__.py:34-148).  lambda is one more forward scan over the
# time-reversed sequence with coefficient A[t+1]^H and zero initial state.


def _shifted_states(zi: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """h[t-1] for every t: the initial state followed by all but the last output."""
    return torch.cat([zi.unsqueeze(1), y[:, :-1]], dim=1)


def _recur_composite(A, zi, y, gy, needs):
    # scalar LPV: A [B, T] or shared [T]
    coef = torch.roll(A.conj_physical(), -1, dims=-1).flip(-1)
    lam = torch.ops.philtorch.recur(coef, torch.zeros_like(zi), gy.flip(1)).flip(1)
    gA = gzi = gx = None
    if needs[1]:
        gzi = A.conj_physical()[..., 0] * lam[:, 0]
    if needs[2]:
        gx = lam
    if needs[0]:
        per_step = lam * _shifted_states(zi, y).conj_physical()
        gA = per_step if A.dim() == 2 else per_step.sum(0)
    return gA, gzi, gx


def _recurN_composite(A, zi, y, gy, needs):
    # LPV M x M: A [B, T, M, M] or shared [T, M, M]
    AH = A.mT.conj_physical()
    coef = torch.roll(AH, -1, dims=-3).flip(-3)
    lam = MatrixOps.recur(coef, torch.zeros_like(zi), gy.flip(1)).flip(1)
    gA = gzi = gx = None
    if needs[1]:
        gzi = (AH[..., 0, :, :] @ lam[:, 0, :, None]).squeeze(-1)
    if needs[2]:
        gx = lam
    if needs[0]:
        per_step = lam.unsqueeze(-1) * _shifted_states(zi, y).conj_physical().unsqueeze(-2)
        gA = per_step if A.dim() == 4 else per_step.sum(0)
    return gA, gzi, gx


def _lti_recur_composite(A, zi, y, gy, needs):
    # scalar LTI: A [B] (per row) or a single shared value
    a_conj = A.conj_physical()
    lam = torch.ops.philtorch.lti_recur(a_conj, torch.zeros_like(zi), gy.flip(1)).flip(1)
    gA = gzi = gx = None
    batched = A.dim() == 1 and A.numel() == gy.size(0)
    if needs[1]:
        gzi = lam[:, 0] * (a_conj if batched else a_conj.reshape(()))
    if needs[2]:
        gx = lam
    if needs[0]:
        per_row = torch.linalg.vecdot(_shifted_states(zi, y), lam)  # sum_t conj(h[t-1]) lambda[t]
        gA = per_row if batched else per_row.sum().reshape(A.shape)
    return gA, gzi, gx


def _lti_recurN_composite(A, zi, y, gy, needs):
    # LTI M x M: A [B, M, M] or shared [M, M]
    AH = A.mT.conj_physical()
    lam = MatrixOps.lti_recur(AH, torch.zeros_like(zi), gy.flip(1)).flip(1)
    gA = gzi = gx = None
    if needs[1]:
        gzi = (AH @ lam[:, 0, :, None]).squeeze(-1)
    if needs[2]:
        gx = lam
    if needs[0]:
        hp = _shifted_states(zi, y).conj_physical()
        per_row = lam.mT @ hp  # [B, M, M]: sum_t lambda[t] conj(h[t-1])^T
        gA = per_row if A.dim() == 3 else per_row.sum(0)
    return gA, gzi, gx


class MatrixOps:
    """Routes an M x M scan to the op the reference would call for that M."""

    @staticmethod
    def recur(A, zi, x):
        if x.size(-1) == 2:
            return torch.ops.philtorch.recur2(A, zi, x)
        return torch.ops.philtorch.recurN(A, zi, x)

    @staticmethod
    def lti_recur(A, zi, x):
        if x.size(-1) == 2:
            return torch.ops.philtorch.lti_recur2(A, zi, x)
        return torch.ops.philtorch.lti_recurN(A, zi, x)


def _setup_context(ctx: Any, inputs: tuple, output: torch.Tensor) -> None:
    A, zi, _ = inputs
    ctx.save_for_backward(A, zi, output)


def _make_backward(fused_name: str, composite):
    def backward(ctx: Any, grad_y: torch.Tensor):
        A, zi, y = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if torch.is_grad_enabled():
            gA, gzi, gx = composite(A, zi, y, grad_y, needs)
        else:
            fused = getattr(torch.ops.philtorch, fused_name)
            gA, gzi, gx = fused(A, zi, y, grad_y)
        return (gA if needs[0] else None, gzi if needs[1] else None, gx if needs[2] else None)

    return backward


if EXTENSION_LOADED:

    def _fake_like(x):
        return torch.empty_like(x, memory_format=torch.contiguous_format)

    @torch.library.register_fake("philtorch::recur")
    def _(A, zi, x):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(A.ndim in (1, 2), lambda: "A must be 1D (shared) or 2D.")
        torch._check(A.shape[-1] == x.shape[1], lambda: "A's last dimension must match x's time dimension")
        torch._check(zi.ndim == 1 and zi.shape[0] == x.shape[0], lambda: "x and zi must have the same batch size.")
        if A.ndim == 2:
            torch._check(A.shape[0] == x.shape[0], lambda: "If A is 2D, its first dimension must match x's batch size.")
        return _fake_like(x)

    def _fake_recurN(A, zi, x, square2: bool):
        if square2:
            torch._check(A.shape[-1] == A.shape[-2] == 2, lambda: "A must be square.")
        else:
            torch._check(A.shape[-1] == A.shape[-2] == x.shape[2], lambda: "A must be square.")
        torch._check(A.ndim in (3, 4), lambda: "A must be 3D or 4D.")
        torch._check(zi.shape[1] == x.shape[2], lambda: "zi's last dimension must match x's.")
        torch._check(x.shape[1] == A.shape[-3], lambda: "x's second dimension must match A's last-3 dimension.")
        torch._check(x.shape[0] == zi.shape[0], lambda: "x and zi must have the same batch size.")
        if A.ndim == 4:
            torch._check(A.shape[0] == x.shape[0], lambda: "If A is 4D, its first dimension must match x's batch size.")
        return _fake_like(x)

    def _fake_lti_recurN(A, zi, x, square2: bool):
        if square2:
            torch._check(A.shape[-1] == A.shape[-2] == 2, lambda: "A must be square.")
        else:
            torch._check(A.shape[-1] == A.shape[-2] == x.shape[2], lambda: "A must be square.")
        torch._check(A.ndim in (2, 3), lambda: "A must be 2D or 3D.")
        torch._check(zi.shape[1] == x.shape[2], lambda: "zi's last dimension must match x's.")
        torch._check(x.shape[0] == zi.shape[0], lambda: "x and zi must have the same batch size.")
        if A.ndim == 3:
            torch._check(A.shape[0] == x.shape[0], lambda: "If A is 3D, its first dimension must match x's batch size.")
        return _fake_like(x)

    torch.library.register_fake("philtorch::recur2")(lambda A, zi, x: _fake_recurN(A, zi, x, True))
    torch.library.register_fake("philtorch::recurN")(lambda A, zi, x: _fake_recurN(A, zi, x, False))
    torch.library.register_fake("philtorch::lti_recur2")(lambda A, zi, x: _fake_lti_recurN(A, zi, x, True))
    torch.library.register_fake("philtorch::lti_recurN")(lambda A, zi, x: _fake_lti_recurN(A, zi, x, False))

    @torch.library.register_fake("philtorch::lti_recur")
    def _(A, zi, x):
        torch._check(A.ndim <= 1, lambda: "A must be 1D or scalar.")
        torch._check(zi.shape[0] == x.shape[0], lambda: "x and zi must have the same batch size.")
        if A.ndim == 1 and A.shape[0] != 1:
            torch._check(A.shape[0] == x.shape[0], lambda: "If A is 1D, its length must match x's batch size.")
        return _fake_like(x)

    def _fake_backward(A, zi, y, grad_y):
        return _fake_like(A), _fake_like(zi), _fake_like(y)

    for _name in ("recur_backward", "recurN_backward", "lti_recur_backward", "lti_recurN_backward"):
        torch.library.register_fake(f"philtorch::{_name}")(_fake_backward)

    for _op, _fused, _comp in (
        ("recur", "recur_backward", _recur_composite),
        ("recur2", "recurN_backward", _recurN_composite),
        ("recurN", "recurN_backward", _recurN_composite),
        ("lti_recur", "lti_recur_backward", _lti_recur_composite),
        ("lti_recur2", "lti_recurN_backward", _lti_recurN_composite),
        ("lti_recurN", "lti_recurN_backward", _lti_recurN_composite),
    ):
        torch.library.register_autograd(
            f"philtorch::{_op}", _make_backward(_fused, _comp), setup_context=_setup_context
        )


def _has_op(name: str) -> bool:
    try:
        getattr(torch.ops.philtorch, name)
        return True
    except (AttributeError, RuntimeError):
        return False


def _op_ctx(*tensors):
    """The context of a philtorch op call: as it is where autograd records a
    graph (grad mode on and an input wanting a gradient); else below the
    Autograd dispatch key, which skips the Python layer of the op's
    registered autograd (torch.library) on every call."""
    import contextlib

    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        return contextlib.nullcontext()
    return torch._C._AutoDispatchBelowAutograd()


# (a _C.so built before the cascade ops existed lacks them; the in-tree build
# imports this package before it rebuilds that library)
def _n_ckpt(x, T):
    """Forward state checkpoints per row and section of the cascade ops."""
    every = 32 if x.dtype == torch.float32 else 8
    return (T + every - 1) // every


if EXTENSION_LOADED and _has_op("sosfilt"):
    # fused cascade of second-order sections: (y, zf, ckpt); ckpt holds the
    # forward's state checkpoints (fp64 pairs, every 32nd step for float32
    # and every 8th for float64: the gradient backward's lane chunks)
    @torch.library.register_fake("philtorch::sosfilt")
    def _(sos, zi, x):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(sos.ndim in (2, 3) and sos.shape[-1] == 6, lambda: "sos must be (sections, 6) or (batch, sections, 6)")
        torch._check(1 <= sos.shape[-2] <= 8, lambda: "1 to 8 sections per call")
        if sos.ndim == 3:
            torch._check(sos.shape[0] == x.shape[0], lambda: "a 3D sos must have x's batch size")
        B, T, S = x.shape[0], x.shape[1], sos.shape[-2]
        if zi is not None:
            torch._check(tuple(zi.shape) == (B, S, 2), lambda: "zi must be (batch, sections, 2)")
        return (_fake_like(x), x.new_empty((B, S, 2)), x.new_empty((B, S, _n_ckpt(x, T), 2), dtype=torch.float64))

    @torch.library.register_fake("philtorch::sosfilt_backward")
    def _(sos, x, ckpt, grad_y, grad_zf, need_sos):
        return _fake_like(x), sos.new_empty(sos.shape), x.new_empty((x.shape[0], sos.shape[-2], 2))

    def _sosfilt_setup(ctx, inputs, output):
        sos, zi, x = inputs
        ctx.save_for_backward(sos, x, output[2], zi)
        ctx.has_zi = zi is not None
        ctx.set_materialize_grads(False)  # no zero gradients for the checkpoints or an unused zf

    def _sosfilt_composite(sos, zi, x, gy, gzf, needs):
        """Gradient through the per-section lfilter(tdf2) chain on the native
        2x2 scan ops, whose own backward is differentiable: used under
        create_graph (double backward)."""
        from .lti.filtering import _sosfilt_sections

        wrt = [t for t, n in zip((sos, zi, x), needs) if n and t is not None]
        with torch.enable_grad():
            zb = zi if zi is not None else x.new_zeros(x.size(0), sos.size(-2), 2)
            y, zf = _sosfilt_sections(sos, x, zb, unroll_factor=1)
            outs, grads = [y], [gy]
            if gzf is not None:
                outs.append(zf)
                grads.append(gzf)
            res = list(torch.autograd.grad(outs, wrt, grads, create_graph=True, allow_unused=True))
        out = []
        for t, n in zip((sos, zi, x), needs):
            g = res.pop(0) if (n and t is not None) else None
            out.append(torch.zeros_like(t) if (g is None and n and t is not None) else g)
        return tuple(out)

    def _sosfilt_backward(ctx, gy, gzf, _gckpt):
        sos, x, ckpt, zi = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if gy is None:
            gy = torch.zeros_like(x)
        if torch.is_grad_enabled():  # create_graph: a differentiable gradient
            return _sosfilt_composite(sos, zi, x, gy, gzf, needs)
        need_sos = bool(needs[0])
        with _op_ctx(sos, x, gy):
            gx, gsos, gzi = torch.ops.philtorch.sosfilt_backward(sos, x, ckpt, gy, gzf, need_sos)
        return (gsos if needs[0] else None, gzi if ctx.has_zi and needs[1] else None, gx if needs[2] else None)

    torch.library.register_autograd("philtorch::sosfilt", _sosfilt_backward, setup_context=_sosfilt_setup)

if EXTENSION_LOADED and _has_op("biquad"):
    # one biquad from lfilter's b and a on the cascade kernel: (y, zf, ckpt)
    @torch.library.register_fake("philtorch::biquad")
    def _(b, a, zi, x):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(b.ndim == a.ndim and b.ndim in (1, 2), lambda: "b and a must both be 1D or both 2D")
        torch._check(1 <= b.shape[-1] <= 3 and a.shape[-1] == 2, lambda: "a biquad")
        B, T = x.shape
        return _fake_like(x), x.new_empty((B, 2)), x.new_empty((B, 1, _n_ckpt(x, T), 2), dtype=torch.float64)

    @torch.library.register_fake("philtorch::biquad_backward")
    def _(b, a, x, ckpt, grad_y, grad_zf, need_coef):
        return [_fake_like(x), b.new_empty(b.shape), a.new_empty(a.shape), x.new_empty((x.shape[0], 2))]

    def _biquad_setup(ctx, inputs, output):
        b, a, zi, x = inputs
        ctx.save_for_backward(b, a, x, output[2], zi)
        ctx.has_zi = zi is not None
        # the checkpoints and an unused final state need no zero gradients
        ctx.set_materialize_grads(False)

    def _biquad_backward(ctx, gy, gzf, _gckpt):
        """philtorch::biquad_backward: the cascade kernel's adjoint pass at
        one section, with the coefficient sums where b or a needs a
        gradient.  Under create_graph: the gradient of the section as
        philtorch's lfilter composes it (a differentiable composite)."""
        b, a, x, ckpt, zi = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if gy is None:
            gy = torch.zeros_like(x)
        if torch.is_grad_enabled():
            sos = torch.cat([torch.nn.functional.pad(b, (0, 3 - b.size(-1))), torch.ones_like(a[..., :1]), a],
                            dim=-1).unsqueeze(-2)
            zs = None if zi is None else zi.unsqueeze(1)
            res = _sosfilt_composite(sos, zs, x, gy, None if gzf is None else gzf.unsqueeze(1),
                                     (needs[0] or needs[1], needs[2], needs[3]))
            gsos, gz, gx = res
            gb = ga = None
            if gsos is not None:
                gb = gsos[..., 0, : b.size(-1)]
                ga = gsos[..., 0, 4:6]
            return (gb if needs[0] else None, ga if needs[1] else None,
                    gz[:, 0] if (gz is not None and ctx.has_zi and needs[2]) else None, gx if needs[3] else None)
        need_coef = bool(needs[0] or needs[1])
        with _op_ctx(b, a, x, gy):
            gx, gb, ga, gzi = torch.ops.philtorch.biquad_backward(b, a, x, ckpt, gy, gzf, need_coef)
        return (gb if needs[0] else None, ga if needs[1] else None, gzi if ctx.has_zi and needs[2] else None,
                gx if needs[3] else None)

    torch.library.register_autograd("philtorch::biquad", _biquad_backward, setup_context=_biquad_setup)

if EXTENSION_LOADED and _has_op("biquad_cols"):
    # biquad with b and a as columns of coefficient tables (col -1: b or a
    # itself): the backward writes the tables' gradients whole, the column's
    # in place and zeros elsewhere
    def _table_col(t, col):
        return t if col < 0 else t.select(-2, col)

    @torch.library.register_fake("philtorch::biquad_cols")
    def _(bt, b_col, at, a_col, zi, x):
        b, a = _table_col(bt, b_col), _table_col(at, a_col)
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(b.ndim == a.ndim and b.ndim in (1, 2), lambda: "b and a must both be 1D or both 2D")
        torch._check(1 <= b.shape[-1] <= 3 and a.shape[-1] == 2, lambda: "a biquad")
        B, T = x.shape
        return _fake_like(x), x.new_empty((B, 2)), x.new_empty((B, 1, _n_ckpt(x, T), 2), dtype=torch.float64)

    @torch.library.register_fake("philtorch::biquad_cols_backward")
    def _(bt, b_col, at, a_col, x, ckpt, grad_y, grad_zf, need_coef):
        return [_fake_like(x), bt.new_empty(bt.shape), at.new_empty(at.shape), x.new_empty((x.shape[0], 2))]

    def _biquad_cols_setup(ctx, inputs, output):
        bt, b_col, at, a_col, zi, x = inputs
        ctx.save_for_backward(bt, at, x, output[2], zi)
        ctx.cols = (b_col, a_col)
        ctx.has_zi = zi is not None
        ctx.set_materialize_grads(False)

    def _biquad_cols_grads(bt, b_col, at, a_col, x, ckpt, zi, has_zi, needs, gy, gzf):
        """(grad bt, grad at, grad zi, grad x) of philtorch::biquad_cols for
        `needs` (bt, at, zi, x): biquad_backward whose coefficient gradients
        are the tables' (the caller's b[:, s] costs autograd no zero-filled
        table and column copy), called below the Autograd dispatch key.
        Under create_graph: the section's composite gradient scattered into
        the table's column."""
        if gy is None:
            gy = torch.zeros_like(x)
        if torch.is_grad_enabled():
            b, a = _table_col(bt, b_col), _table_col(at, a_col)
            sos = torch.cat([torch.nn.functional.pad(b, (0, 3 - b.size(-1))), torch.ones_like(a[..., :1]), a],
                            dim=-1).unsqueeze(-2)
            zs = None if zi is None else zi.unsqueeze(1)
            gsos, gz, gx = _sosfilt_composite(sos, zs, x, gy, None if gzf is None else gzf.unsqueeze(1),
                                              (needs[0] or needs[1], needs[2], needs[3]))
            gbt = gat = None
            if gsos is not None:
                gb, ga = gsos[..., 0, : b.size(-1)], gsos[..., 0, 4:6]
                gbt = gb if b_col < 0 else torch.select_scatter(torch.zeros_like(bt), gb, -2, b_col)
                gat = ga if a_col < 0 else torch.select_scatter(torch.zeros_like(at), ga, -2, a_col)
            return (gbt if needs[0] else None, gat if needs[1] else None,
                    gz[:, 0] if (gz is not None and has_zi and needs[2]) else None, gx if needs[3] else None)
        need_coef = bool(needs[0] or needs[1])
        with torch._C._AutoDispatchBelowAutograd():
            gx, gbt, gat, gzi = torch.ops.philtorch.biquad_cols_backward(bt, b_col, at, a_col, x, ckpt, gy, gzf,
                                                                         need_coef)
        return (gbt if needs[0] else None, gat if needs[1] else None, gzi if has_zi and needs[2] else None,
                gx if needs[3] else None)

    def _biquad_cols_backward(ctx, gy, gzf, _gckpt):
        bt, at, x, ckpt, zi = ctx.saved_tensors
        b_col, a_col = ctx.cols
        n = ctx.needs_input_grad  # bt, b_col, at, a_col, zi, x
        gbt, gat, gzi, gx = _biquad_cols_grads(bt, b_col, at, a_col, x, ckpt, zi, ctx.has_zi,
                                               (n[0], n[2], n[4], n[5]), gy, gzf)
        return gbt, None, gat, None, gzi, gx

    class _BiquadColumns(torch.autograd.Function):
        """lfilter's route for a biquad whose b or a is a column of a
        coefficient table: philtorch::biquad_cols and its backward, called
        below the Autograd dispatch key.  The op's own registered autograd
        (torch.library) runs the same gradients; this Function skips that
        layer's Python per call (about half of the C4 caller pattern's host
        time per lfilter, where the step is bound by the host)."""

        @staticmethod
        def forward(ctx, bt, at, zi, x, b_col, a_col):
            with torch._C._AutoDispatchBelowAutograd():
                y, zf, ckpt = torch.ops.philtorch.biquad_cols(bt, b_col, at, a_col, zi, x)
            ctx.save_for_backward(bt, at, x, ckpt, zi)
            ctx.cols = (b_col, a_col)
            ctx.has_zi = zi is not None
            ctx.set_materialize_grads(False)
            return y, zf

        @staticmethod
        def backward(ctx, gy, gzf):
            bt, at, x, ckpt, zi = ctx.saved_tensors
            b_col, a_col = ctx.cols
            n = ctx.needs_input_grad  # bt, at, zi, x, b_col, a_col
            gbt, gat, gzi, gx = _biquad_cols_grads(bt, b_col, at, a_col, x, ckpt, zi, ctx.has_zi,
                                                   (n[0], n[1], n[2], n[3]), gy, gzf)
            return gbt, gat, gzi, gx, None, None

    torch.library.register_autograd("philtorch::biquad_cols", _biquad_cols_backward,
                                    setup_context=_biquad_cols_setup)

if EXTENSION_LOADED and _has_op("filtfilt"):
    # zero-phase filter of order 4 at most (lti.filtfilt's fused route); its
    # gradients are philtorch::filtfilt_backward
    def _filtfilt_fake_check(b, a, x, padlen):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(b.ndim == a.ndim and b.ndim in (1, 2), lambda: "b and a must both be 1D or both 2D")
        torch._check(1 <= b.shape[-1] <= 5 and 1 <= a.shape[-1] <= 4, lambda: "order 4 at most")
        torch._check(0 <= padlen < x.shape[1], lambda: "0 <= padlen < T")

    @torch.library.register_fake("philtorch::filtfilt")
    def _(b, a, x, padmode, padlen):
        _filtfilt_fake_check(b, a, x, padlen)
        return _fake_like(x)

    if _has_op("filtfilt_backward"):
        @torch.library.register_fake("philtorch::filtfilt_backward")
        def _(b, a, x, grad_y, padmode, padlen, need_coef, mid=None, h1=None, h2=None):
            _filtfilt_fake_check(b, a, grad_y, padlen)
            if need_coef:
                return [_fake_like(grad_y), b.new_empty(b.shape), a.new_empty(a.shape)]
            return [_fake_like(grad_y), b.new_empty((0,)), a.new_empty((0,))]

        class _FiltfiltAdjoint(torch.autograd.Function):
            """grad_x = J^T grad_y of filtfilt (b and a constant), whose own
            gradient is J ggx: filtfilt again (second order)."""

            @staticmethod
            def forward(ctx, b, a, gy, padmode, padlen):
                ctx.save_for_backward(b, a)
                ctx.pad = (padmode, padlen)
                return torch.ops.philtorch.filtfilt_backward(b, a, gy, gy, padmode, padlen, False)[0]

            @staticmethod
            def backward(ctx, ggx):
                b, a = ctx.saved_tensors
                return None, None, torch.ops.philtorch.filtfilt(b, a, ggx, *ctx.pad), None, None

        def _filtfilt_setup(ctx, inputs, output):
            b, a, x, padmode, padlen = inputs
            # filtfilt_states: pass 1's output and both passes' states too
            kept = tuple(output[1:]) if isinstance(output, (tuple, list)) else ()
            for t in kept:
                ctx.mark_non_differentiable(t)
            ctx.save_for_backward(b, a, x, *kept)
            ctx.pad = (padmode, padlen)
            ctx.set_materialize_grads(False)

        def _filtfilt_backward(ctx, gy):
            """x only: J^T gy (philtorch::filtfilt_backward, differentiable
            again through filtfilt).  b or a too: the same op's coefficient
            mode; under create_graph, the gradient of the composed route the
            kernels replace (pad, lfilter_zi, two lfilter passes;
            philtorch/lti/filtering.py:413-484), recomputed from the inputs."""
            needs = ctx.needs_input_grad
            if gy is None or not any(needs[:3]):
                return None, None, None, None, None
            saved = ctx.saved_tensors
            b, a, x = saved[:3]
            kept = saved[3:]  # mid, h1, h2 from filtfilt_states, or none
            need_coef = bool(needs[0] or needs[1])
            if not need_coef:
                if torch.is_grad_enabled():
                    return None, None, _FiltfiltAdjoint.apply(b, a, gy, *ctx.pad), None, None
                with _op_ctx(b, a, x, gy):
                    gx = torch.ops.philtorch.filtfilt_backward(b, a, x, gy, *ctx.pad, False)[0]
                return None, None, gx, None, None
            if torch.is_grad_enabled():
                from .lti.filtering import _PAD_CODES, _filtfilt_composed

                padmode = {v: k for k, v in _PAD_CODES.items()}[ctx.pad[0]]
                inputs = (b, a, x)
                wrt = [i for i in range(3) if needs[i]]
                with torch.enable_grad():
                    y = _filtfilt_composed(b, a, x, padmode, ctx.pad[1], unroll_factor=1)
                    res = torch.autograd.grad(y, [inputs[i] for i in wrt], gy, create_graph=True, allow_unused=True)
                out = [None] * 5
                for i, g in zip(wrt, res):
                    out[i] = g if g is not None else torch.zeros_like(inputs[i])
                return tuple(out)
            with _op_ctx(b, a, x, gy):
                gx, gb, ga = torch.ops.philtorch.filtfilt_backward(b, a, x, gy, *ctx.pad, True, *kept)
            return gb if needs[0] else None, ga if needs[1] else None, gx if needs[2] else None, None, None

        torch.library.register_autograd("philtorch::filtfilt", _filtfilt_backward, setup_context=_filtfilt_setup)

        if _has_op("filtfilt_states"):

            @torch.library.register_fake("philtorch::filtfilt_states")
            def _(b, a, x, padmode, padlen):
                _filtfilt_fake_check(b, a, x, padlen)
                B, T = x.shape
                M = max(b.shape[-1] - 1, a.shape[-1])
                al = lambda n: (n + 255) // 256 * 256  # noqa: E731  (the library's 256-byte alignment)
                mid = al(B * T * x.element_size()) + al(B * 4 * x.element_size()) if B else 0
                return (_fake_like(x), x.new_empty((mid,), dtype=torch.uint8), x.new_empty((B, T, M)),
                        x.new_empty((B, T, M)))

            def _filtfilt_states_backward(ctx, gy, gmid, gh1, gh2):
                """filtfilt's backward with pass 1's output and both passes'
                states from the forward (not differentiable): the coefficient
                mode skips computing them again."""
                return _filtfilt_backward(ctx, gy)

            torch.library.register_autograd("philtorch::filtfilt_states", _filtfilt_states_backward,
                                            setup_context=_filtfilt_setup)

if EXTENSION_LOADED and _has_op("lti_ss"):
    # single-input single-output LTI state space of order <= 4: (y, zf)
    @torch.library.register_fake("philtorch::lti_ss")
    def _(A, B, C, D, zi, x, out_idx, reverse=False):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(A.ndim in (2, 3) and A.shape[-1] == A.shape[-2], lambda: "A must be (M, M) or (batch, M, M)")
        return _fake_like(x), x.new_empty((x.shape[0], A.shape[-1]))

    if _has_op("lti_ss_backward"):

        @torch.library.register_fake("philtorch::lti_ss_backward")
        def _(A, B, C, D, zi, x, grad_y, grad_zf, out_idx, reverse=False, hs=None):
            e = lambda t: x.new_empty(t.shape) if t is not None else x.new_empty((0,))  # noqa: E731
            return [e(A), e(B), e(C), e(D), x.new_empty((x.shape[0], A.shape[-1])), _fake_like(x)]

    def _lti_ss_setup(ctx, inputs, output):
        A, B, C, D, zi, x, out_idx = inputs[:7]
        ctx.out_idx = out_idx
        ctx.reverse = bool(inputs[7]) if len(inputs) > 7 else False
        # lti_ss_states: the forward's states too, for the coefficient backward
        hs = output[2] if len(output) > 2 else None
        if hs is not None:
            ctx.mark_non_differentiable(hs)
        ctx.save_for_backward(A, B, C, D, zi, x, hs)
        ctx.set_materialize_grads(False)

    def _lti_ss_backward(ctx, gy, gzf):
        """With A, B, C, D constant: the adjoint model (A^T, input vector C,
        output vector B, D) run in the opposite time direction from dL/dzf
        gives grad_x and grad_zi in one more lti_ss pass (the reversed mode
        for a forward call and the other way round: no flipped copies).
        With a coefficient gradient wanted: philtorch::lti_ss_backward, the
        forward again keeping its states, then the adjoint pass summing
        lambda h^T, lambda x, g h and g x.  Under create_graph: the gradient
        of the composite the fused kernel replaces (B x, the native scan,
        the state shift, C h + D x; philtorch/lti/ssm.py:386-589),
        recomputed from the inputs and differentiable again."""
        from .lti.ssm import _state_space_composite

        saved = ctx.saved_tensors
        inputs, hs = saved[:6], saved[6]
        needs = ctx.needs_input_grad
        A, B, C, D, zi, x = inputs
        if any(needs[:4]) and not torch.is_grad_enabled() and _has_op("lti_ss_backward"):
            g = gy if gy is not None else torch.zeros_like(x)
            with _op_ctx(A, B, C, D, zi, x, g):
                res = torch.ops.philtorch.lti_ss_backward(A, B, C, D, zi, x, g, gzf, ctx.out_idx, ctx.reverse, hs)
            out = [None] * 8
            for i, t in enumerate(inputs[:5] + (x,)):
                if t is not None and needs[i]:
                    out[i] = res[i]
            return tuple(out)
        if not any(needs[:4]):
            M = A.size(-1)
            unit = lambda i: torch.nn.functional.one_hot(torch.tensor(i, device=x.device), M).to(x.dtype)  # noqa: E731
            g = gy if gy is not None else torch.zeros_like(x)
            with _op_ctx(A, B, C, D, gzf, g):
                gx, gzi = torch.ops.philtorch.lti_ss(A.mT.contiguous(), C if C is not None else unit(ctx.out_idx),
                                                     B if B is not None else unit(0), D, gzf, g, 0, not ctx.reverse)
            return (None, None, None, None, gzi if zi is not None and needs[4] else None,
                    gx if needs[5] else None, None, None)
        wrt = [i for i, t in enumerate(inputs) if t is not None and needs[i]]
        create = torch.is_grad_enabled()  # create_graph, read before enable_grad
        with torch.enable_grad():
            if ctx.reverse:
                y, zf = _state_space_composite(A, B, C, D, zi, x.flip(-1), out_idx=ctx.out_idx)
                y = y.flip(-1)
            else:
                y, zf = _state_space_composite(*inputs, out_idx=ctx.out_idx)
            outs, grads = [y], [gy if gy is not None else torch.zeros_like(y)]
            if gzf is not None:
                outs.append(zf)
                grads.append(gzf)
            res = torch.autograd.grad(outs, [inputs[i] for i in wrt], grads, create_graph=create,
                                      allow_unused=True)
        out = [None] * 8
        for i, g in zip(wrt, res):
            out[i] = g if g is not None else torch.zeros_like(inputs[i])
        return tuple(out)

    torch.library.register_autograd("philtorch::lti_ss", _lti_ss_backward, setup_context=_lti_ss_setup)

    if _has_op("lti_ss_states"):

        @torch.library.register_fake("philtorch::lti_ss_states")
        def _(A, B, C, D, zi, x, out_idx, reverse=False):
            torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
            M = A.shape[-1]
            return _fake_like(x), x.new_empty((x.shape[0], M)), x.new_empty((x.shape[0], x.shape[1], M))

        def _lti_ss_states_backward(ctx, gy, gzf, ghs):
            """lti_ss's backward with the states the forward kept (hs is not
            differentiable): the coefficient backward runs its adjoint pass
            only."""
            return _lti_ss_backward(ctx, gy, gzf)

        torch.library.register_autograd("philtorch::lti_ss_states", _lti_ss_states_backward,
                                        setup_context=_lti_ss_setup)

if EXTENSION_LOADED and _has_op("lfilter_ss"):
    # lfilter of order <= 4 from b and a in one pass: (y, zf)
    @torch.library.register_fake("philtorch::lfilter_ss")
    def _(b, a, zi, x, form, reverse=False):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        M = max(b.shape[-1] - 1, a.shape[-1])
        torch._check(1 <= M <= 4, lambda: "filters of order 1 to 4")
        return _fake_like(x), x.new_empty((x.shape[0], M))

    if _has_op("lfilter_ss_backward"):

        @torch.library.register_fake("philtorch::lfilter_ss_backward")
        def _(b, a, zi, x, grad_y, grad_zf, form, reverse=False, hs=None):
            M = max(b.shape[-1] - 1, a.shape[-1])
            return [b.new_empty(b.shape), a.new_empty(a.shape), x.new_empty((x.shape[0], M)), _fake_like(x)]

    def _lfilter_ss_setup(ctx, inputs, output):
        b, a, zi, x, form = inputs[:5]
        ctx.form = form
        ctx.reverse = bool(inputs[5]) if len(inputs) > 5 else False
        # lfilter_ss_states: the forward's states too, for the coefficient backward
        hs = output[2] if len(output) > 2 else None
        if hs is not None:
            ctx.mark_non_differentiable(hs)
        ctx.save_for_backward(b, a, zi, x, hs)
        ctx.set_materialize_grads(False)

    def _lfilter_ss_backward(ctx, gy, gzf):
        """With b and a constant: the adjoint of a companion-form filter is
        the other companion form of the same filter run in the opposite time
        direction (TDF-II <-> DF-II: A^T, with the input and output vectors
        swapped), from dL/dzf, so grad_x and grad_zi are one more lfilter_ss
        pass (the reversed mode for a forward call and the other way round:
        no flipped copies).  With a gradient of b or a wanted:
        philtorch::lfilter_ss_backward (the forward again keeping its
        states, the adjoint pass with the model's gradient sums, the chain
        rule to b and a).  Under create_graph: the gradient of the
        companion-form route the kernel replaces (philtorch/lti/
        filtering.py:273-333), recomputed from the inputs."""
        from .lti.filtering import _ssm_lfilter

        saved = ctx.saved_tensors
        b, a, zi, x = inputs = saved[:4]
        hs = saved[4]
        needs = ctx.needs_input_grad
        if (needs[0] or needs[1]) and not torch.is_grad_enabled() and _has_op("lfilter_ss_backward"):
            g = gy if gy is not None else torch.zeros_like(x)
            with _op_ctx(b, a, zi, x, g):
                gb, ga, gzi, gx = torch.ops.philtorch.lfilter_ss_backward(b, a, zi, x, g, gzf, ctx.form, ctx.reverse,
                                                                          hs)
            return (gb if needs[0] else None, ga if needs[1] else None,
                    gzi if zi is not None and needs[2] else None, gx if needs[3] else None, None, None)
        if not (needs[0] or needs[1]):
            g = gy if gy is not None else torch.zeros_like(x)
            with _op_ctx(b, a, gzf, g):
                gx, gzi = torch.ops.philtorch.lfilter_ss(b, a, gzf, g, 1 - ctx.form, not ctx.reverse)
            return (None, None, gzi if zi is not None and needs[2] else None, gx if needs[3] else None, None, None)
        wrt = [i for i, t in enumerate(inputs) if t is not None and needs[i]]
        create = torch.is_grad_enabled()  # create_graph, read before enable_grad
        with torch.enable_grad():
            z = zi if zi is not None else x.new_zeros(x.size(0), max(b.size(-1) - 1, a.size(-1)))
            xs = x.flip(-1) if ctx.reverse else x
            y, zf = _ssm_lfilter(b, a, xs, z, form=("tdf2", "df2")[ctx.form], unroll_factor=1)
            if ctx.reverse:
                y = y.flip(-1)
            outs, grads = [y], [gy if gy is not None else torch.zeros_like(y)]
            if gzf is not None:
                outs.append(zf)
                grads.append(gzf)
            res = torch.autograd.grad(outs, [inputs[i] for i in wrt], grads, create_graph=create,
                                      allow_unused=True)
        out = [None] * 6
        for i, g in zip(wrt, res):
            out[i] = g if g is not None else torch.zeros_like(inputs[i])
        return tuple(out)

    torch.library.register_autograd("philtorch::lfilter_ss", _lfilter_ss_backward, setup_context=_lfilter_ss_setup)

    if _has_op("lfilter_ss_states"):

        @torch.library.register_fake("philtorch::lfilter_ss_states")
        def _(b, a, zi, x, form, reverse=False):
            torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
            M = max(b.shape[-1] - 1, a.shape[-1])
            return _fake_like(x), x.new_empty((x.shape[0], M)), x.new_empty((x.shape[0], x.shape[1], M))

        def _lfilter_ss_states_backward(ctx, gy, gzf, ghs):
            """lfilter_ss's backward with the states the forward kept (hs is
            not differentiable): the gradients of b and a take the adjoint
            pass only."""
            return _lfilter_ss_backward(ctx, gy, gzf)

        torch.library.register_autograd("philtorch::lfilter_ss_states", _lfilter_ss_states_backward,
                                        setup_context=_lfilter_ss_setup)

if EXTENSION_LOADED and _has_op("lpv_ss"):
    # single-input single-output LPV state space of order <= 4: (y, zf)
    @torch.library.register_fake("philtorch::lpv_ss")
    def _(A, B, C, D, zi, x, out_idx, reverse=False, transpose_A=False):
        torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
        torch._check(A.ndim in (3, 4) and A.shape[-1] == A.shape[-2], lambda: "A must be (T, M, M) or (batch, T, M, M)")
        return _fake_like(x), x.new_empty((x.shape[0], A.shape[-1]))

    if _has_op("lpv_ss_backward"):

        @torch.library.register_fake("philtorch::lpv_ss_backward")
        def _(A, B, C, D, zi, x, grad_y, grad_zf, out_idx, reverse=False, transpose_A=False, hs=None):
            e = lambda t: x.new_empty(t.shape) if t is not None else x.new_empty((0,))  # noqa: E731
            return [e(A), e(B), e(C), e(D), x.new_empty((x.shape[0], A.shape[-1])), _fake_like(x)]

    def _lpv_ss_setup(ctx, inputs, output):
        A, B, C, D, zi, x, out_idx = inputs[:7]
        ctx.out_idx = out_idx
        ctx.reverse = bool(inputs[7]) if len(inputs) > 7 else False
        ctx.transpose_A = bool(inputs[8]) if len(inputs) > 8 else False
        # lpv_ss_states: the forward's states too, for the coefficient backward
        hs = output[2] if len(output) > 2 else None
        if hs is not None:
            ctx.mark_non_differentiable(hs)
        ctx.save_for_backward(A, B, C, D, zi, x, hs)
        ctx.set_materialize_grads(False)

    def _lpv_ss_backward(ctx, gy, gzf):
        """With A, B, C, D constant: the adjoint model (A[t]^T, input vector
        c[t], output vector b[t], d[t]) run in the opposite time direction
        from dL/dzf gives grad_x and grad_zi in one more lpv_ss pass, which
        reads A transposed where it lies (transpose_A; no copy of A).  With
        a coefficient gradient wanted: philtorch::lpv_ss_backward (the
        forward again keeping its states, then the adjoint pass writing
        lambda[t+1] h[t]^T, lambda[t+1] x[t], g[t] h[t], g[t] x[t] per step,
        summed over the axes an operand shares).  Under create_graph, or
        where the fused backward's per-row step gradients of operands the
        rows share would exceed lpv.ssm._LPV_ROW_SCRATCH_LIMIT: the gradient
        of the composite the fused kernel replaces (B x, the native LPV
        scan, the state shift, C h + D x; philtorch/lpv/ssm.py:337-581),
        recomputed from the inputs (and differentiable again)."""
        from .lpv import ssm as _lpv_ssm

        _lpv_state_space_composite = _lpv_ssm._lpv_state_space_composite
        saved = ctx.saved_tensors
        inputs, hs = saved[:6], saved[6]
        needs = ctx.needs_input_grad
        A, B, C, D, zi, x = inputs
        out = [None] * 9
        # the fused backward, unless its per-row step gradients of shared
        # operands would exceed _LPV_ROW_SCRATCH_LIMIT (then the composite)
        fits = _lpv_ssm._lpv_row_scratch_bytes(A, B, C, D, x, needs[:4]) <= _lpv_ssm._LPV_ROW_SCRATCH_LIMIT
        if any(needs[:4]) and not torch.is_grad_enabled() and _has_op("lpv_ss_backward") and fits:
            g = gy if gy is not None else torch.zeros_like(x)
            with _op_ctx(A, B, C, D, zi, x, g):
                res = torch.ops.philtorch.lpv_ss_backward(A, B, C, D, zi, x, g, gzf, ctx.out_idx, ctx.reverse,
                                                          ctx.transpose_A, hs)
            for i, t in enumerate(inputs):
                if t is not None and needs[i]:
                    out[i] = res[i]
            return tuple(out)
        if not any(needs[:4]):
            M = A.size(-1)
            c_in = C
            if C is None:
                c_in = x.new_zeros(1, 1, M)
                c_in[..., ctx.out_idx] = 1
            g = gy if gy is not None else torch.zeros_like(x)
            with _op_ctx(A, c_in, B, D, gzf, g):
                gx, gzi = torch.ops.philtorch.lpv_ss(A, c_in, B, D, gzf, g, 0, not ctx.reverse,
                                                  not ctx.transpose_A)
            if zi is not None and needs[4]:
                out[4] = gzi
            if needs[5]:
                out[5] = gx
            return tuple(out)
        wrt = [i for i, t in enumerate(inputs) if t is not None and needs[i]]
        if not wrt:
            return tuple(out)
        create = torch.is_grad_enabled()  # create_graph, read before enable_grad
        with torch.enable_grad():
            Am = A.mT if ctx.transpose_A else A  # the model's matrices
            if ctx.reverse:
                # the forward model over the time-flipped row and operands
                ft = lambda t, d: t if t is None or t.size(d) == 1 else t.flip(d)  # noqa: E731
                y, zf = _lpv_state_space_composite(Am.flip(-3), ft(B, 1), ft(C, 1), ft(D, 1), zi, x.flip(-1),
                                                   out_idx=ctx.out_idx)
                y = y.flip(-1)
            else:
                y, zf = _lpv_state_space_composite(Am, B, C, D, zi, x, out_idx=ctx.out_idx)
            outs, grads = [y], [gy if gy is not None else torch.zeros_like(y)]
            if gzf is not None:
                outs.append(zf)
                grads.append(gzf)
            res = torch.autograd.grad(outs, [inputs[i] for i in wrt], grads, create_graph=create,
                                      allow_unused=True)
        for i, g in zip(wrt, res):
            out[i] = g if g is not None else torch.zeros_like(inputs[i])
        return tuple(out)

    torch.library.register_autograd("philtorch::lpv_ss", _lpv_ss_backward, setup_context=_lpv_ss_setup)

    if _has_op("lpv_ss_states"):

        @torch.library.register_fake("philtorch::lpv_ss_states")
        def _(A, B, C, D, zi, x, out_idx, reverse=False, transpose_A=False):
            torch._check(x.ndim == 2, lambda: "x must be 2D (batch, time)")
            M = A.shape[-1]
            return _fake_like(x), x.new_empty((x.shape[0], M)), x.new_empty((x.shape[0], x.shape[1], M))

        def _lpv_ss_states_backward(ctx, gy, gzf, ghs):
            """lpv_ss's backward with the states the forward kept (hs is not
            differentiable): the coefficient backward runs its adjoint pass
            only, instead of the forward again first."""
            return _lpv_ss_backward(ctx, gy, gzf)

        torch.library.register_autograd("philtorch::lpv_ss_states", _lpv_ss_states_backward,
                                        setup_context=_lpv_ss_setup)

if EXTENSION_LOADED and _has_op("mimo_ss"):
    # LTI state space with F inputs and P outputs per step (F, P <= 4): (y, zf)
    @torch.library.register_fake("philtorch::mimo_ss")
    def _(A, B, C, D, zi, x, reverse=False):
        torch._check(x.ndim == 3, lambda: "x must be 3D (batch, time, features)")
        torch._check(A.ndim in (2, 3) and A.shape[-1] == A.shape[-2], lambda: "A must be (M, M) or (batch, M, M)")
        torch._check(C.ndim in (2, 3), lambda: "C must be (P, M) or (batch, P, M)")
        return x.new_empty((x.shape[0], x.shape[1], C.shape[-2])), x.new_empty((x.shape[0], A.shape[-1]))

    def _mimo_ss_setup(ctx, inputs, output):
        ctx.reverse = bool(inputs[6]) if len(inputs) > 6 else False
        ctx.save_for_backward(*inputs[:6])
        ctx.set_materialize_grads(False)

    if _has_op("mimo_ss_grad_sums"):

        @torch.library.register_fake("philtorch::mimo_ss_grad_sums")
        def _(lam, hs, x, g, shared, want, Bm=None, Dm=None):
            st = lam if lam is not None else hs
            M = st.shape[2] if st is not None else 1
            dims = ((M, M), (M, x.shape[2]), (g.shape[2], M), (g.shape[2], x.shape[2]))
            out = [x.new_empty(((1 if (shared >> i) & 1 else x.shape[0]),) + dims[i]) if (want >> i) & 1
                   else x.new_empty((0,)) for i in range(4)]
            if shared & 16 and want & 1:  # A per step
                out[0] = x.new_empty((x.shape[0], x.shape[1], M, M))
            if want & 16:  # the input's gradient
                out.append(x.new_empty(x.shape))
            return out

    def _mimo_ss_backward(ctx, gy, gzf):
        """The adjoint model (A^T, input matrix C^T, output matrix B^T, D^T)
        run in the opposite time direction from dL/dzf gives grad_x and
        grad_zi in one more mimo_ss pass; where the coefficient gradients
        take the adjoint states (A or B wanted), their pass gives grad_zi and
        the sums pass writes grad_x = B^T lambda[t+1] + D^T g[t] instead.
        The coefficient gradients
            dL/dA = sum_t lambda[t+1] h[t]^T,  dL/dB = sum_t lambda[t+1] x[t]^T,
            dL/dC = sum_t g[t] h[t]^T,         dL/dD = sum_t g[t] x[t]^T
        take the states h[t] (the forward again with C = I and no D) and the
        adjoint states lambda[t+1] (the adjoint pass with output matrix I),
        each one more mimo_ss pass, and philtorch::mimo_ss_grad_sums: the
        four sums over time (and the rows, for a shared operand) in one pass
        over lambda, h, x and g.  Under create_graph: the gradient
        of the composite the fused kernel replaces (B x, the native scan,
        the state shift, C h + D x; philtorch/lti/ssm.py:386-589),
        recomputed from the inputs and differentiable again."""
        from .lti.ssm import _mimo_composite

        inputs = ctx.saved_tensors
        A, B, C, D, zi, x = inputs
        needs = ctx.needs_input_grad
        out = [None] * 7
        if torch.is_grad_enabled():  # create_graph
            wrt = [i for i, t in enumerate(inputs) if t is not None and needs[i]]
            with torch.enable_grad():
                y, zf = _mimo_composite(*inputs, reverse=ctx.reverse)
                outs, grads = [y], [gy if gy is not None else torch.zeros_like(y)]
                if gzf is not None:
                    outs.append(zf)
                    grads.append(gzf)
                res = torch.autograd.grad(outs, [inputs[i] for i in wrt], grads, create_graph=True,
                                          allow_unused=True)
            for i, g in zip(wrt, res):
                out[i] = g if g is not None else torch.zeros_like(inputs[i])
            return tuple(out)
        M = A.size(-1)
        g = gy if gy is not None else x.new_zeros(x.size(0), x.size(1), C.size(-2))
        At, Ct = A.mT.contiguous(), C.mT.contiguous()
        eye = torch.eye(M, dtype=x.dtype, device=x.device)
        # lambda is wanted for A or B: its pass also gives grad_zi, and the
        # sums pass writes grad_x = B^T lambda + D^T g beside the sums
        lam_pass = needs[0] or needs[1]
        with _op_ctx():
            if not lam_pass and (needs[5] or (needs[4] and zi is not None)):
                gx, gzi = torch.ops.philtorch.mimo_ss(At, Ct, B.mT.contiguous(),
                                                      D.mT.contiguous() if D is not None else None, gzf, g,
                                                      not ctx.reverse)
                out[5] = gx if needs[5] else None
                out[4] = gzi if needs[4] and zi is not None else None
            hs = lam = None
            if needs[0] or needs[2]:
                hs, _ = torch.ops.philtorch.mimo_ss(A, B, eye, None, zi, x, ctx.reverse)
            if lam_pass:
                lam, gzi = torch.ops.philtorch.mimo_ss(At, Ct, eye, None, gzf, g, not ctx.reverse)
                out[4] = gzi if needs[4] and zi is not None else None
        want = sum(1 << i for i in range(4) if needs[i] and inputs[i] is not None)
        if lam_pass and needs[5]:
            want |= 16
        if want:
            shared = sum(1 << i for i, t in enumerate((A, B, C, D)) if t is not None and t.dim() == 2)
            with _op_ctx():
                sums = torch.ops.philtorch.mimo_ss_grad_sums(lam, hs, x, g, shared, want, B, D)
            for i in range(4):
                if (want >> i) & 1:
                    out[i] = sums[i][0] if (shared >> i) & 1 else sums[i]
            if want & 16:
                out[5] = sums[4]
        return tuple(out)

    torch.library.register_autograd("philtorch::mimo_ss", _mimo_ss_backward, setup_context=_mimo_ss_setup)

if EXTENSION_LOADED and _has_op("lpv_mimo_ss"):
    # LPV state space (A[t]) with F inputs and P outputs per step (F, P <= 4),
    # B, C, D constant in time: (y, zf)
    @torch.library.register_fake("philtorch::lpv_mimo_ss")
    def _(A, B, C, D, zi, x, reverse=False, transpose_A=False):
        torch._check(x.ndim == 3, lambda: "x must be 3D (batch, time, features)")
        torch._check(A.ndim in (3, 4) and A.shape[-1] == A.shape[-2], lambda: "A must be (T, M, M) or (batch, T, M, M)")
        torch._check(C.ndim in (2, 3), lambda: "C must be (P, M) or (batch, P, M)")
        return x.new_empty((x.shape[0], x.shape[1], C.shape[-2])), x.new_empty((x.shape[0], A.shape[-1]))

    def _lpv_mimo_ss_setup(ctx, inputs, output):
        ctx.reverse = bool(inputs[6]) if len(inputs) > 6 else False
        ctx.transpose_A = bool(inputs[7]) if len(inputs) > 7 else False
        # lpv_mimo_ss_states: the forward's states too, for the coefficient backward
        hs = output[2] if len(output) > 2 else None
        if hs is not None:
            ctx.mark_non_differentiable(hs)
        ctx.save_for_backward(*inputs[:6], hs)
        ctx.set_materialize_grads(False)

    def _lpv_mimo_ss_backward(ctx, gy, gzf):
        """The adjoint model (A[t]^T read in place, input matrix C^T, output
        matrix B^T, D^T) in the opposite time direction from dL/dzf gives
        grad_x and grad_zi in one more lpv_mimo_ss pass (where the
        coefficient gradients take the adjoint states, their pass gives
        grad_zi and the sums pass grad_x = B^T lambda[t+1] + D^T g[t]).
        The coefficients: the states h[t] (the forward again with C = I, no
        D) and the adjoint states lambda[t+1] (the adjoint pass with output
        matrix I), then one pass of philtorch::mimo_ss_grad_sums writing
        dL/dA[t] = lambda[t+1] h[t]^T per step (summed over the rows after,
        for a shared A) and summing lambda x^T, g h^T, g x^T over time for
        B, C, D.  Under create_graph: the gradient of the composite the fused kernel replaces (B x, the native
        LPV scan, the state shift, C h + D x; philtorch/lpv/ssm.py:337-581),
        recomputed from the inputs and differentiable again."""
        from .lpv.ssm import _lpv_mimo_composite

        saved = ctx.saved_tensors
        inputs, kept_hs = saved[:6], saved[6]
        A, B, C, D, zi, x = inputs
        needs = ctx.needs_input_grad
        out = [None] * 8
        if torch.is_grad_enabled():  # create_graph
            wrt = [i for i, t in enumerate(inputs) if t is not None and needs[i]]
            with torch.enable_grad():
                y, zf = _lpv_mimo_composite(*inputs, reverse=ctx.reverse, transpose_A=ctx.transpose_A)
                outs, grads = [y], [gy if gy is not None else torch.zeros_like(y)]
                if gzf is not None:
                    outs.append(zf)
                    grads.append(gzf)
                res = torch.autograd.grad(outs, [inputs[i] for i in wrt], grads, create_graph=True,
                                          allow_unused=True)
            for i, g in zip(wrt, res):
                out[i] = g if g is not None else torch.zeros_like(inputs[i])
            return tuple(out)
        M = A.size(-1)
        g = gy if gy is not None else x.new_zeros(x.size(0), x.size(1), C.size(-2))
        Ct = C.mT.contiguous()
        eye = torch.eye(M, dtype=x.dtype, device=x.device)
        rev, tr = ctx.reverse, ctx.transpose_A
        op = torch.ops.philtorch.lpv_mimo_ss
        # lambda is wanted for A[t] or B: its pass also gives grad_zi, and
        # the sums pass writes grad_x = B^T lambda + D^T g beside the sums
        lam_pass = needs[0] or needs[1]
        with _op_ctx():
            if not lam_pass and (needs[5] or (needs[4] and zi is not None)):
                gx, gzi = op(A, Ct, B.mT.contiguous(), D.mT.contiguous() if D is not None else None, gzf, g,
                             not rev, not tr)
                out[5] = gx if needs[5] else None
                out[4] = gzi if needs[4] and zi is not None else None
            hs = lam = None
            if needs[0] or needs[2]:
                # the forward's states, kept by lpv_mimo_ss_states or computed again
                hs = kept_hs if kept_hs is not None else op(A, B, eye, None, zi, x, rev, tr)[0]
            if lam_pass:
                lam, gzi = op(A, Ct, eye, None, gzf, g, not rev, not tr)
                out[4] = gzi if needs[4] and zi is not None else None
            want = sum(1 << i for i in (0, 1, 2, 3) if needs[i] and inputs[i] is not None)
            if lam_pass and needs[5]:
                want |= 16
            if want:
                shared = sum(1 << i for i, t in enumerate((A, B, C, D)) if i > 0 and t is not None and t.dim() == 2)
                shared |= 16 | (32 if tr else 0)  # dL/dA[t] per step (transposed for A[t]^T)
                sums = torch.ops.philtorch.mimo_ss_grad_sums(lam, hs, x, g, shared, want, B, D)
                if want & 1:
                    out[0] = sums[0].sum(0) if A.dim() == 3 else sums[0]
                for i in (1, 2, 3):
                    if (want >> i) & 1:
                        out[i] = sums[i][0] if (shared >> i) & 1 else sums[i]
                if want & 16:
                    out[5] = sums[4]
        return tuple(out)

    torch.library.register_autograd("philtorch::lpv_mimo_ss", _lpv_mimo_ss_backward,
                                    setup_context=_lpv_mimo_ss_setup)

    if _has_op("lpv_mimo_ss_states"):

        @torch.library.register_fake("philtorch::lpv_mimo_ss_states")
        def _(A, B, C, D, zi, x, reverse=False, transpose_A=False):
            M = A.shape[-1]
            return (x.new_empty((x.shape[0], x.shape[1], C.shape[-2])), x.new_empty((x.shape[0], M)),
                    x.new_empty((x.shape[0], x.shape[1], M)))

        def _lpv_mimo_ss_states_backward(ctx, gy, gzf, ghs):
            """lpv_mimo_ss's backward with the states the forward kept (hs is
            not differentiable): no states pass."""
            return _lpv_mimo_ss_backward(ctx, gy, gzf)

        torch.library.register_autograd("philtorch::lpv_mimo_ss_states", _lpv_mimo_ss_states_backward,
                                        setup_context=_lpv_mimo_ss_setup)

from . import mat  # noqa: E402,F401
from . import lti  # noqa: E402,F401
from . import lpv  # noqa: E402,F401
