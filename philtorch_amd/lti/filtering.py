"""IIR filtering on the LTI state-space layer (philtorch/lti/filtering.py).

``lfilter`` builds the companion-form state-space model of ``b / a`` and runs
it through ``state_space`` (transposed direct form II by default), so with
``unroll_factor=1`` on a HIP device every filter is one native scan
(``philtorch::lti_recur2`` for a biquad); a biquad in TDF-II form runs the
fused cascade kernel instead (Bx, scan, state shift and output in one pass),
unless forward-mode AD is active; every other filter of order <= 4 with no
gradient wanted runs philtorch::lfilter_ss (the companion model built inside
the kernel).  ``filtfilt`` and ``lfilter_zi`` follow the
reference and SciPy; a biquad ``filtfilt`` with no gradient wanted runs both
passes in philtorch::filtfilt.  Cascaded second-order sections are composed by the
caller, one ``lfilter`` per section, as in the reference (it has no SOS API),
or all at once by ``sosfilt``, which on a HIP device runs the whole cascade in
one fused kernel per direction.
"""
from __future__ import annotations

from functools import partial
from typing import Optional, Union

import torch
import torch.nn.functional as F
from torch import Tensor

from ..mat import companion
from .ssm import state_space


def lfilter_zi(a: Tensor, b: Optional[Tensor] = None, transpose: bool = True) -> Tensor:
    """Steady-state initial conditions of ``b / a`` for a unit step
    (philtorch/lti/filtering.py:107-142; scipy.signal.lfilter_zi for the TDF-II
    form).  ``a`` holds the denominator without its leading 1."""
    assert a.dim() >= 1, "Denominator coefficients a must be at least 1D."
    if not transpose:
        n = a.size(-1) + 1
        A = companion(a)
        Bv = a.new_zeros(n - 1)
        Bv[0] = 1.0
    elif b is not None:
        assert b.dim() >= 1, "Numerator coefficients b must be at least 1D."
        n = max(b.size(-1), a.size(-1) + 1)
        if b.size(-1) < n:
            b = F.pad(b, (0, n - b.size(-1)))
        if a.size(-1) < n - 1:
            a = F.pad(a, (0, n - 1 - a.size(-1)))
        A = companion(a).mT.conj()
        Bv = b[..., 1:] - b[..., :1] * a
    else:
        raise ValueError("Numerator coefficients b must be provided for transpose=True.")
    I_minus_A = torch.eye(n - 1, device=a.device, dtype=a.dtype) - A
    if I_minus_A.ndim == 2 and Bv.ndim > 1:
        I_minus_A = I_minus_A.expand(*Bv.shape[:-1], -1, -1)
    return torch.linalg.solve(I_minus_A, Bv)


def _ssm_lfilter(b: Tensor, a: Tensor, x: Tensor, zi: Optional[Tensor] = None, form: str = "df2", **kwargs):
    """Companion-form state-space realisation (philtorch/lti/filtering.py:273-333)."""
    if b.size(-1) < a.size(-1) + 1:
        b = F.pad(b, (0, a.size(-1) + 1 - b.size(-1)))
    elif b.size(-1) > a.size(-1) + 1:
        a = F.pad(a, (0, b.size(-1) - a.size(-1) - 1))
    A = companion(a)
    b0 = b[..., :1]
    if form == "df2":
        filt = partial(state_space, A, B=None, C=b[..., 1:] - b0 * a, D=b[..., 0], zi=zi, out_idx=None, **kwargs)
    elif form == "tdf2":
        filt = partial(state_space, A.mT.conj(), B=(b[..., 1:] - b0 * a).conj(), C=None, D=b[..., 0].conj(),
                       zi=zi, out_idx=0, **kwargs)
    elif form in ("df1", "tdf1"):
        raise NotImplementedError(f"form={form!r} (an FIR stage around the recursion) is not part of this build")
    else:
        raise ValueError(f"Unknown filter form: {form}")
    return filt(x)


def _fused_biquad_applies(b: Tensor, a: Tensor, x: Tensor, zi: Optional[Tensor], form: str, kwargs) -> bool:
    """A second-order TDF-II filter on a HIP device with the native route
    requested (``unroll_factor=1``): the fused cascade kernel computes the same
    filter in one pass (Bx, the scan, the state shift and C h + D x), with
    first- and second-order reverse-mode gradients.  Forward-mode AD keeps the
    reference's route."""
    from .. import EXTENSION_LOADED

    if not (EXTENSION_LOADED and x.is_cuda and form == "tdf2" and set(kwargs) == {"unroll_factor"}
            and kwargs["unroll_factor"] == 1):
        return False
    if a.size(-1) != 2 or b.size(-1) > 3 or x.dtype not in (torch.float32, torch.float64):
        return False
    if b.dtype != x.dtype or a.dtype != x.dtype or (zi is not None and zi.dtype != x.dtype):
        return False
    if b.dim() != a.dim() or (b.dim() == 2 and not (b.size(0) == a.size(0) == x.size(0))):
        return False
    if zi is not None and not (zi.dim() == 1 or (zi.dim() == 2 and zi.size(0) == x.size(0))):
        return False
    if not hasattr(torch.ops.philtorch, "biquad"):
        return False
    import torch.autograd.forward_ad as fwad

    return all(t is None or fwad.unpack_dual(t).tangent is None for t in (b, a, x, zi))


def _fused_biquad(b: Tensor, a: Tensor, x: Tensor, zi: Optional[Tensor]):
    """lfilter(b, a, x, zi, form="tdf2") of one biquad.  Where b or a needs
    a gradient, the cascade kernel at one section: philtorch::biquad reads b
    and a where they lie (a column of a coefficient table needs no copy) and
    keeps checkpoints for its fused coefficient gradients.  Otherwise the
    state-space kernel (philtorch::lfilter_ss), whose forward and x/zi
    adjoint passes are the shorter ones at one section."""
    if not (torch.is_grad_enabled() and (b.requires_grad or a.requires_grad)) and hasattr(torch.ops.philtorch,
                                                                                          "lfilter_ss"):
        return _fused_lfilter(b, a, x, zi, "tdf2")
    zb = None if zi is None else zi.expand(x.size(0), 2).contiguous()
    bt, b_col = _table_column(b)
    at, a_col = _table_column(a)
    if (b_col >= 0 or a_col >= 0) and hasattr(torch.ops.philtorch, "biquad_cols"):
        # b or a is a column of a coefficient table (the caller's b[:, s]):
        # the table takes its gradient directly
        from .. import _BiquadColumns

        y, zf = _BiquadColumns.apply(bt, at, zb, x, b_col, a_col)
    else:
        from .. import _op_ctx

        with _op_ctx(b, a, zb, x):
            y, zf, _ = torch.ops.philtorch.biquad(b, a, zb, x)
    return y if zi is None else (y, zf)


def _table_column(t: Tensor) -> tuple[Tensor, int]:
    """``(table, s)`` when ``t`` is ``table.select(-2, s)`` of the tensor its
    view chain starts from (the C4 caller's ``b[:, s]`` of a ``(B, S, 3)``
    coefficient table), judged by memory placement; else ``(t, -1)``.

    A column routed this way hands its gradient to the table directly:
    autograd then allocates no zero-filled table and writes no column per
    call (torch's select backward), but the gradient of the column view
    object itself is no longer recorded (``autograd.grad(y, column)`` with
    that very view, its ``retain_grad`` or its hooks).  Views that retain
    their gradient or carry hooks keep the plain route."""
    base = getattr(t, "_base", None)
    if base is None or t.grad_fn is None or not base.requires_grad or t.retains_grad:
        return t, -1
    if getattr(t, "_backward_hooks", None):
        return t, -1
    if base.dim() != t.dim() + 1 or t.dim() not in (1, 2) or base.dtype != t.dtype:
        return t, -1
    if tuple(t.shape) != tuple(base.shape[:-2]) + tuple(base.shape[-1:]):
        return t, -1
    if tuple(t.stride()) != tuple(base.stride()[:-2]) + tuple(base.stride()[-1:]):
        return t, -1
    step = base.stride(-2)
    off = t.storage_offset() - base.storage_offset()
    if step <= 0 or off < 0 or off % step != 0 or off // step >= base.size(-2):
        return t, -1
    return base, off // step


def _fused_lfilter_applies(b: Tensor, a: Tensor, x: Tensor, zi: Optional[Tensor], form: str, kwargs) -> bool:
    """A filter of order 1 to 4 on a HIP device with the native route
    requested (``unroll_factor=1``): philtorch::lfilter_ss builds the
    companion model from b and a inside the kernel and runs B x, the scan,
    the state shift and C h + D x in one pass (the TDF-II biquad takes the
    cascade kernel first); gradients for x and zi are one more pass of the
    adjoint form, those of b and a two fused passes
    (philtorch::lfilter_ss_backward)."""
    from .. import EXTENSION_LOADED

    if not (EXTENSION_LOADED and x.is_cuda and form in ("tdf2", "df2") and set(kwargs) == {"unroll_factor"}
            and kwargs["unroll_factor"] == 1 and x.dim() == 2):
        return False
    M = max(b.size(-1) - 1, a.size(-1))
    if not (1 <= M <= 4 and a.size(-1) >= 1) or x.dtype not in (torch.float32, torch.float64):
        return False
    if b.dtype != x.dtype or a.dtype != x.dtype or (zi is not None and zi.dtype != x.dtype):
        return False
    if b.dim() != a.dim() or (b.dim() == 2 and not (b.size(0) == a.size(0) == x.size(0))):
        return False
    if zi is not None and not (tuple(zi.shape) in ((M,), (x.size(0), M))):
        return False
    if not hasattr(torch.ops.philtorch, "lfilter_ss"):
        return False
    import torch.autograd.forward_ad as fwad

    return all(t is None or fwad.unpack_dual(t).tangent is None for t in (b, a, x, zi))


def _fused_lfilter(b: Tensor, a: Tensor, x: Tensor, zi: Optional[Tensor], form: str):
    """lfilter(b, a, x, zi, form) through philtorch::lfilter_ss."""
    M = max(b.size(-1) - 1, a.size(-1))
    zb = None if zi is None else zi.expand(x.size(0), M).contiguous()
    from .. import _has_op, _op_ctx

    # b or a with a gradient to come: the forward keeps its states
    # (lfilter_ss_states), which their backward would compute again
    keep = torch.is_grad_enabled() and (b.requires_grad or a.requires_grad) and _has_op("lfilter_ss_states")
    with _op_ctx(b, a, zb, x):
        if keep:
            y, zf, _ = torch.ops.philtorch.lfilter_ss_states(b, a, zb, x, 0 if form == "tdf2" else 1)
        else:
            y, zf = torch.ops.philtorch.lfilter_ss(b, a, zb, x, 0 if form == "tdf2" else 1)
    return y if zi is None else (y, zf)


def lfilter(
    b: Tensor,
    a: Tensor,
    x: Tensor,
    zi: Optional[Tensor] = None,
    form: str = "tdf2",
    backend: str = "ssm",
    **kwargs,
) -> Union[Tensor, tuple[Tensor, Tensor]]:
    """Batch of IIR filters ``b / a`` (``a`` without its leading 1)
    (philtorch/lti/filtering.py:211-270).

    Args:
        b: ``(B, M_b+1)`` or ``(M_b+1,)`` numerator.
        a: ``(B, M_a)`` or ``(M_a,)`` denominator after the leading 1.
        x: ``(B, N)`` or ``(N,)`` input.
        zi: optional initial state; when given, ``(y, zf)`` is returned.
        form: ``"tdf2"`` (default) or ``"df2"``.
        backend: ``"ssm"``.
        **kwargs: forwarded to ``state_space`` (e.g. ``unroll_factor=1`` for
            the native scan).
    """
    squeeze_first = x.dim() == 1 and b.dim() == 1 and a.dim() == 1 and (zi is None or zi.dim() == 1)
    if x.dim() == 1:
        x = x.unsqueeze(0)
    elif x.dim() > 2:
        raise ValueError("Input signal x must be 1D or 2D.")
    assert b.dim() in (1, 2), "Numerator coefficients b must be 1D or 2D."
    assert a.dim() in (1, 2), "Denominator coefficients a must be 1D or 2D."
    if backend != "ssm":
        raise ValueError(f"Unknown backend: {backend}")
    if _fused_biquad_applies(b, a, x, zi, form, kwargs):
        y = _fused_biquad(b, a, x, zi)
    elif _fused_lfilter_applies(b, a, x, zi, form, kwargs):
        y = _fused_lfilter(b, a, x, zi, form)
    else:
        y = _ssm_lfilter(b, a, x, zi, form=form, **kwargs)
    if isinstance(y, tuple):
        y, zf = y
        if squeeze_first:
            y, zf = y.squeeze(0), zf.squeeze(0)
        return y, zf
    return y.squeeze(0) if squeeze_first else y


# torch.nn.functional.pad modes with a fused filtfilt (PHS_PAD_* codes)
_PAD_CODES = {"constant": 0, "replicate": 1, "reflect": 2, "circular": 3}


def _fused_filtfilt_applies(b: Tensor, a: Tensor, x: Tensor, padmode: Optional[str], form: str, kwargs) -> bool:
    """A filter of order 4 at most on a HIP device with the native route
    requested (``unroll_factor=1``): philtorch::filtfilt runs both passes
    with the padding, the flips and the trim folded in, and its gradients
    (x, b, a) philtorch::filtfilt_backward.  Its output is the same for the
    ``tdf2`` and ``df2`` forms (each pass starts from the steady state of the
    same transfer function)."""
    from .. import EXTENSION_LOADED

    if not (EXTENSION_LOADED and x.is_cuda and form in ("tdf2", "df2") and set(kwargs) == {"unroll_factor"}
            and kwargs["unroll_factor"] == 1):
        return False
    if padmode is not None and padmode not in _PAD_CODES:
        return False
    if not (1 <= a.size(-1) <= 4 and 1 <= b.size(-1) <= 5) or x.dtype not in (torch.float32, torch.float64):
        return False
    if b.dtype != x.dtype or a.dtype != x.dtype or x.dim() not in (1, 2):
        return False
    if b.dim() != a.dim() or b.dim() not in (1, 2):
        return False
    if b.dim() == 2 and not (x.dim() == 2 and b.size(0) == a.size(0) == x.size(0)):
        return False
    if not hasattr(torch.ops.philtorch, "filtfilt"):
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in (b, a, x)) and not hasattr(torch.ops.philtorch,
                                                                                          "filtfilt_backward"):
        return False
    import torch.autograd.forward_ad as fwad

    return all(fwad.unpack_dual(t).tangent is None for t in (b, a, x))


def _filtfilt_composed(b: Tensor, a: Tensor, x: Tensor, padmode: Optional[str], edge: int, form: str = "tdf2",
                       **kwargs) -> Tensor:
    """The reference's filtfilt steps (philtorch/lti/filtering.py:462-484):
    pad, lfilter_zi, an lfilter pass from zi * ext[:, :1], a second over the
    flipped output from zi * y[:, -1:], the trim and the flip back (each pass
    on the fused lfilter route where it applies)."""
    if edge > 0 and padmode is not None:
        ext = F.pad(x.view(-1, x.size(-1)), (edge, edge), mode=padmode)
        if x.dim() == 1:
            ext = ext.squeeze(0)
    else:
        ext = x
    zi = lfilter_zi(a, b, transpose=(form == "tdf2"))
    y, _ = lfilter(b, a, ext, zi=zi * ext[..., :1], form=form, **kwargs)
    y, _ = lfilter(b, a, y.flip(-1), zi=zi * y[..., -1:], form=form, **kwargs)
    if edge > 0:
        y = y[..., edge:-edge]
    return y.flip(-1)


def _fused_filtfilt(b: Tensor, a: Tensor, x: Tensor, padmode: Optional[str], edge: int) -> Tensor:
    """filtfilt of a filter of order 4 at most through philtorch::filtfilt."""
    x2 = x.reshape(-1, x.size(-1))
    code = _PAD_CODES[padmode] if padmode is not None else 0
    from .. import _has_op, _op_ctx

    # b or a with a gradient to come: the forward keeps pass 1's output and
    # both passes' states (filtfilt_states), which their backward would
    # compute again
    keep = torch.is_grad_enabled() and (b.requires_grad or a.requires_grad) and _has_op("filtfilt_states")
    with _op_ctx(b, a, x2):
        if keep:
            y = torch.ops.philtorch.filtfilt_states(b, a, x2, code, edge if padmode is not None else 0)[0]
        else:
            y = torch.ops.philtorch.filtfilt(b, a, x2, code, edge if padmode is not None else 0)
    return y.reshape(x.shape)


def filtfilt(
    b: Tensor,
    a: Tensor,
    x: Tensor,
    padmode: Optional[str] = "replicate",
    padlen: Optional[int] = None,
    method: str = "pad",
    irlen: Optional[int] = None,
    form: str = "tdf2",
    **kwargs,
) -> Tensor:
    """Zero-phase filtering: a forward and a reversed ``lfilter`` pass with
    edge padding and steady-state initial conditions
    (philtorch/lti/filtering.py:413-484).  A filter of order 4 at most on a
    HIP device with ``unroll_factor=1`` and no gradient wanted runs
    philtorch::filtfilt (two state-space passes, the second in reversed time,
    their entry states derived in the kernel: no padded copy, no flips and no
    host synchronisation; gradients w.r.t. x, b and a through
    philtorch::filtfilt_backward); otherwise the passes are composed as in
    the reference, each pass on the fused lfilter route."""
    assert method in ("pad", "gust"), "Method must be either 'pad' or 'gust'."
    if method == "gust":
        raise NotImplementedError("Gustafsson's method is not implemented yet.")
    if padmode is None:
        padlen = 0
    ntaps = max(b.size(-1), a.size(-1) + 1)
    edge = 3 * ntaps if padlen is None else padlen
    assert x.size(-1) > edge, f"Input signal length {x.size(-1)} must be greater than pad length {edge}."
    if _fused_filtfilt_applies(b, a, x, padmode, form, kwargs):
        return _fused_filtfilt(b, a, x, padmode, edge)
    return _filtfilt_composed(b, a, x, padmode, edge, form, **kwargs)


# sections per fused launch (the backward keeps every section's lane states in LDS)
_SOS_SECTIONS_PER_CALL = 8


def sosfilt(sos: Tensor, x: Tensor, zi: Optional[Tensor] = None, **kwargs) -> Union[Tensor, tuple[Tensor, Tensor]]:
    """Cascade of second-order sections with ``scipy.signal.sosfilt``'s
    semantics (transposed direct form II, filtering along the last axis).

    philtorch has no cascade API; its users chain one ``lfilter(b, a, y,
    form="tdf2")`` per section (philtorch/lti/filtering.py:211-333), which is
    what this computes.  On a HIP device every group of up to 8 sections
    runs in one fused kernel per direction (``philtorch::sosfilt``):
    the intermediate sections' signals never reach memory.  Elsewhere it
    takes that per-section ``lfilter`` route (``**kwargs`` are forwarded to it,
    e.g. ``unroll_factor``).

    Args:
        sos: ``(S, 6)`` or ``(B, S, 6)`` rows ``(b0, b1, b2, a0, a1, a2)``;
            every section is normalised by its ``a0``.
        x: ``(N,)`` or ``(B, N)`` input.
        zi: optional initial states in scipy's layout, ``(S, 2)`` for a 1D
            ``x`` or ``(S, B, 2)``; when given, ``(y, zf)`` is returned with
            ``zf`` in the same layout.
    """
    assert sos.dim() in (2, 3) and sos.size(-1) == 6, "sos must be (sections, 6) or (batch, sections, 6)."
    assert x.dim() in (1, 2), "Input signal x must be 1D or 2D."
    squeeze = x.dim() == 1
    xb = x.unsqueeze(0) if squeeze else x
    batch, S = xb.size(0), sos.size(-2)
    if sos.dim() == 3:
        assert sos.size(0) == batch, "A 3D sos must have x's batch size."
    sos = sos / sos[..., 3:4]
    zb = None
    if zi is not None:
        want = (S, 2) if squeeze else (S, batch, 2)
        assert tuple(zi.shape) == want, f"zi must have shape {want}, got {tuple(zi.shape)}"
        zb = (zi.unsqueeze(1) if squeeze else zi).transpose(0, 1)  # (B, S, 2)
    if xb.is_cuda:
        y, zf = _sosfilt_fused(sos, xb, zb)
    else:
        y, zf = _sosfilt_sections(sos, xb, zb, **kwargs)
    if squeeze:
        y = y.squeeze(0)
    if zi is None:
        return y
    zf = zf.transpose(0, 1)
    return y, (zf.squeeze(1) if squeeze else zf)


def _sosfilt_fused(sos: Tensor, x: Tensor, zi: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    from .. import require_extension

    require_extension()
    dtype = x.dtype
    if dtype in (torch.float16, torch.bfloat16):
        x, sos = x.float(), sos.float()
        zi = None if zi is None else zi.float()
    else:
        sos = sos.to(dtype)
    from .. import _op_ctx

    y, zfs = x, []
    for s0 in range(0, sos.size(-2), _SOS_SECTIONS_PER_CALL):
        part = sos[..., s0:s0 + _SOS_SECTIONS_PER_CALL, :]
        zpart = None if zi is None else zi[:, s0:s0 + part.size(-2)].contiguous()
        with _op_ctx(part, zpart, y):
            y, zf, _ = torch.ops.philtorch.sosfilt(part.contiguous(), zpart, y.contiguous())
        zfs.append(zf)
    return y.to(dtype), torch.cat(zfs, dim=1).to(dtype)


def _sosfilt_sections(sos: Tensor, x: Tensor, zi: Optional[Tensor], **kwargs) -> tuple[Tensor, Tensor]:
    """One lfilter(tdf2) per section on the reference's state-space route."""
    y, zfs = x, []
    for s in range(sos.size(-2)):
        b, a = sos[..., s, 0:3], sos[..., s, 4:6]
        z = x.new_zeros(x.size(0), 2) if zi is None else zi[:, s]
        y, zf = _ssm_lfilter(b, a, y, z, form="tdf2", **kwargs)
        zfs.append(zf)
    return y, torch.stack(zfs, dim=1)
