"""Scalar LTI recurrence ``h[t] = a h[t-1] + x[t]`` (philtorch/lti/recur.py).

``LTIRecurrence`` is the autograd Function over ``philtorch::lti_recur``
(reference philtorch/lti/recur.py:8-78).  ``linear_recurrence`` is the
pure-PyTorch route (per-step loop, or a two-level blocked scan when
``unroll_factor > 1``) that the reference keeps for use without the
extension (philtorch/lti/recur.py:94-192).
"""
from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.autograd import Function


class LTIRecurrence(Function):
    """Autograd Function of the native scalar LTI scan.

    forward : ``torch.ops.philtorch.lti_recur(a, init, x)``; ``a`` is a scalar,
              ``[1]`` or ``[B]``; ``init`` is ``[B]``; ``x`` is ``[B, T]``.
    backward: the adjoint scan.  Without ``create_graph`` one fused kernel
              (``lti_recur_backward``) produces every gradient; with it, the
              composite formula re-enters this Function so it stays
              differentiable (reference lti/recur.py:25-59).
    jvp     : one more forward scan with input ``dx + h[t-1] da``
              (reference lti/recur.py:61-78).
    """

    @staticmethod
    def forward(a: Tensor, init: Tensor, x: Tensor) -> Tensor:
        return torch.ops.philtorch.lti_recur(a, init, x)

    @staticmethod
    def setup_context(ctx: Any, inputs: tuple, output: Tensor) -> None:
        a, init, _ = inputs
        ctx.save_for_backward(a, init, output)
        ctx.save_for_forward(a, init, output)

    @staticmethod
    def backward(ctx: Any, grad_out: Tensor):
        a, init, out = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if not torch.is_grad_enabled():
            ga, gi, gx = torch.ops.philtorch.lti_recur_backward(a, init, out, grad_out)
            return (ga if needs[0] else None, gi if needs[1] else None, gx if needs[2] else None)

        a_conj = a.conj_physical()
        lam = LTIRecurrence.apply(a_conj, torch.zeros_like(init), grad_out.flip(1)).flip(1)
        grad_a = grad_init = grad_x = None
        batched = a.dim() == 1 and a.numel() == grad_out.size(0)
        if needs[1]:
            grad_init = lam[:, 0] * (a_conj if batched else a_conj.reshape(()))
        if needs[2]:
            grad_x = lam
        if needs[0]:
            prev = torch.cat([init.unsqueeze(1), out[:, :-1]], dim=1)
            per_row = torch.linalg.vecdot(prev, lam)
            grad_a = per_row if batched else per_row.sum().reshape(a.shape)
        return grad_a, grad_init, grad_x

    @staticmethod
    def jvp(ctx: Any, grad_a: Optional[Tensor], grad_init: Optional[Tensor], grad_x: Optional[Tensor]) -> Tensor:
        a, init, out = ctx.saved_tensors
        t_init = grad_init if grad_init is not None else torch.zeros_like(init)
        t_x = grad_x if grad_x is not None else torch.zeros_like(out)
        if grad_a is not None:
            prev = torch.cat([init.unsqueeze(1), out[:, :-1]], dim=1)
            t_x = t_x + prev * grad_a.reshape(-1, 1)
        return LTIRecurrence.apply(a, t_init, t_x)


def _scalar_recursion_loop(a: Tensor, init: Tensor, x: Tensor) -> Tensor:
    h = init
    outs = []
    for xt in x.unbind(dim=1):
        h = a * h + xt
        outs.append(h)
    return torch.stack(outs, dim=1)


def linear_recurrence(a: Tensor, init: Tensor, x: Tensor, *, unroll_factor: int = 1) -> Tensor:
    """Batched scalar LTI recurrence ``h[t] = a h[t-1] + x[t]`` in PyTorch.

    Args:
        a: scalar or ``[B]`` coefficients.
        init: scalar or ``[B]`` initial state.
        x: ``[B, N]`` input.
        unroll_factor: 1 runs the per-step loop; ``k > 1`` runs a two-level
            blocked scan (``k`` vectorised steps inside blocks, a recursive
            scan over block carries).
    Returns:
        ``[B, N]`` states (reference philtorch/lti/recur.py:94-192).
    """
    assert x.dim() == 2, f"Input x must be 2D, got {x.shape}"
    assert a.dim() in (0, 1), f"State matrix a must be 1D or 0D, got {a.shape}"
    if a.dim() == 1 and a.size(0) > 1 and a.size(0) != x.size(0):
        raise ValueError(
            f"State matrix a must be 1D with the same batch size as x, got a: {a.size(0)}, x: {x.size(0)}"
        )
    if a.dim() == 0:
        a = a.expand(1)
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
    if k == 1 or k >= N:
        return _scalar_recursion_loop(a, init, x)

    pad = (-N) % k
    xb = F.pad(x, (0, pad)).unflatten(1, (-1, k))  # [B, n, k]
    a_col = a.reshape(-1, 1, 1)
    # local scans inside each block with a zero carry
    h = torch.zeros_like(xb[..., 0])
    cols = []
    for i in range(k):
        h = a_col[..., 0] * h + xb[..., i]
        cols.append(h)
    local = torch.stack(cols, dim=-1)
    powers = torch.cumprod(a.reshape(-1, 1).expand(-1, k), dim=-1)  # a^1..a^k, [1 or B, k]
    carries = linear_recurrence(powers[:, -1], init, local[..., -1], unroll_factor=k)  # [B, n]
    prev = torch.cat([init.reshape(-1, 1).expand(batch, 1), carries[:, :-1]], dim=1)
    out = local + powers.unsqueeze(1) * prev.unsqueeze(-1)
    out = out.flatten(1, 2)
    return out[:, :N] if pad else out
