"""IIR filtering on the LTI state-space layer (philtorch/lti/filtering.py).

``lfilter`` builds the companion-form state-space model of ``b / a`` and runs
it through ``state_space`` (transposed direct form II by default), so with
``unroll_factor=1`` on a HIP device every biquad section is one native 2x2
scan (``philtorch::lti_recur2``).  ``filtfilt`` and ``lfilter_zi`` follow the
reference and SciPy.  Cascaded second-order sections are composed by the
caller, one ``lfilter`` per section, as in the reference (it has no SOS API).
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
    y = _ssm_lfilter(b, a, x, zi, form=form, **kwargs)
    if isinstance(y, tuple):
        y, zf = y
        if squeeze_first:
            y, zf = y.squeeze(0), zf.squeeze(0)
        return y, zf
    return y.squeeze(0) if squeeze_first else y


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
    (philtorch/lti/filtering.py:413-484)."""
    assert method in ("pad", "gust"), "Method must be either 'pad' or 'gust'."
    if method == "gust":
        raise NotImplementedError("Gustafsson's method is not implemented yet.")
    if padmode is None:
        padlen = 0
    ntaps = max(b.size(-1), a.size(-1) + 1)
    edge = 3 * ntaps if padlen is None else padlen
    assert x.size(-1) > edge, f"Input signal length {x.size(-1)} must be greater than pad length {edge}."
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
