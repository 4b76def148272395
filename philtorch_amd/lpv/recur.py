"""Scalar LPV (time-varying) recurrence ``h[t] = a[t] h[t-1] + x[t]``.

``linear_recurrence`` mirrors philtorch/lpv/recur.py:20-101 (same signature,
checks and errors).  With ``unroll_factor == 1`` on a HIP device it runs the
native single-pass scan ``philtorch::recur`` (differentiable through the
registered fused adjoint kernel); the reference has no native op here and
runs a Python loop of T ``addcmul`` calls.  Elsewhere it keeps the
reference's pure-PyTorch route: the per-step loop, or a two-level blocked
scan when ``unroll_factor > 1``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from .. import EXTENSION_LOADED


def _native_ok(a: Tensor, init: Tensor, x: Tensor) -> bool:
    """The native scan serves CPU and HIP tensors (all on one device)."""
    return EXTENSION_LOADED and (x.is_cpu or x.is_cuda) and a.device == x.device and init.device == x.device


def _scalar_recursion_loop(a: Tensor, init: Tensor, x: Tensor) -> Tensor:
    h = init
    outs = []
    for at, xt in zip(a.unbind(dim=-1), x.unbind(dim=-1)):
        h = torch.addcmul(xt, h, at)
        outs.append(h)
    return torch.stack(outs, dim=-1)


def linear_recurrence(a: Tensor, init: Tensor, x: Tensor, *, unroll_factor: int = 1) -> Tensor:
    """Linear recurrence with time-varying coefficients.

    Args:
        a: ``[N]`` (shared by the batch) or ``[B, N]`` coefficients.
        init: scalar or ``[B]`` initial state.
        x: ``[B, N]`` input.
        unroll_factor: 1 = the native scan (``philtorch::recur``) on CPU and
            HIP tensors alike (the per-step PyTorch loop only without the
            extension); ``k > 1`` = blocked PyTorch scan with blocks of ``k``
            steps.
    Returns:
        ``[B, N]`` states.
    """
    assert x.dim() == 2, f"Input x must be 2D, got {x.shape}"
    assert a.dim() in (1, 2), f"State matrix a must be 1D or 2D, got {a.shape}"
    if a.dim() == 1 and a.size(0) != x.size(1):
        raise ValueError(
            f"State matrix a must be 1D with the same length as x, got a: {a.size(0)}, x: {x.size(1)}"
        )
    batch, N = x.shape
    assert init.dim() in (0, 1), f"Initial state init must be 1D or 0D, got {init.shape}"
    if init.dim() == 1 and init.size(0) > 1 and init.size(0) != batch:
        raise ValueError(
            f"Initial state init must be 1D with the same batch size as x, got init: {init.size(0)}, x: {batch}"
        )
    if init.dim() == 0:
        init = init.expand(1)
    if unroll_factor < 1:
        raise ValueError("Unroll factor must be >= 1")
    k = unroll_factor

    if k == 1 and _native_ok(a, init, x):
        dt = torch.promote_types(torch.promote_types(a.dtype, init.dtype), x.dtype)
        return torch.ops.philtorch.recur(a.to(dt), init.to(dt).expand(batch), x.to(dt))

    if k == 1 or k >= N:
        return _scalar_recursion_loop(a, init, x)

    pad = (-N) % k
    xb = F.pad(x, (0, pad)).unflatten(1, (-1, k))  # [B, n, k]
    ab = F.pad(a, (0, pad)).unflatten(-1, (-1, k))  # [n, k] or [B, n, k]
    h = torch.zeros_like(xb[..., 0])
    cols = []
    for i in range(k):
        h = ab[..., i] * h + xb[..., i]
        cols.append(h)
    local = torch.stack(cols, dim=-1)  # block-local scan from a zero state
    gains = torch.cumprod(ab, dim=-1)  # prod of a over the block prefix
    carries = linear_recurrence(gains[..., -1], init, local[..., -1], unroll_factor=k)  # [B, n]
    prev = torch.cat([init.expand(batch).unsqueeze(1), carries[:, :-1]], dim=1)
    out = (local + gains * prev.unsqueeze(-1)).flatten(1, 2)
    return out[:, :N] if pad else out
