"""Matrix helpers used to build state-space inputs (philtorch/mat.py)."""
from __future__ import annotations

import torch
from torch import Tensor


def companion(a: Tensor) -> Tensor:
    """Companion matrix of the all-pole coefficients ``a`` (shape ``(..., M)``).

    Row 0 holds ``-a``; the sub-diagonal holds ones, so for ``M = 2`` the
    result is ``[[-a1, -a2], [1, 0]]`` (philtorch/mat.py:42-62).
    """
    assert a.dim() >= 1, "All-pole coefficients must be at least 1D."
    M = a.size(-1)
    out = a.new_zeros(a.shape + (M,))
    out[..., 0, :] = -a
    if M > 1:
        idx = torch.arange(M - 1, device=a.device)
        out[..., idx + 1, idx] = 1
    return out
