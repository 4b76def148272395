"""Time-invariant (LTI) state-space recursion and models (philtorch/lti/ssm.py).

``LTIMatrixRecurrence`` is the autograd Function over ``philtorch::lti_recur2``
/ ``philtorch::lti_recurN`` (reference philtorch/lti/ssm.py:43-115).  On a HIP
device with ``unroll_factor`` 1 (or None where the reference keeps None) the
recursion runs as one native scan; elsewhere the reference's pure-PyTorch
routes are kept.  ``diag_state_space`` runs its per-eigenvalue scalar scans
through ``LTIRecurrence`` (the native ``philtorch::lti_recur``).
"""
from __future__ import annotations

from functools import partial
from typing import Any, Optional

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.autograd import Function

from .. import EXTENSION_LOADED, HELION_LOADED
from .recur import LTIRecurrence, linear_recurrence


def extension_backend_indicator(x: Tensor, M: int) -> bool:
    """True when the native matrix scan serves this input: extension loaded,
    state of order M >= 2 (M = 1 goes through ``LTIRecurrence``), on the CPU
    (any order) or on a HIP device (M <= 4).  The reference,
    philtorch/lti/ssm.py:13-25, takes the CPU for M >= 2 and the GPU for
    M = 2 only."""
    return EXTENSION_LOADED and M >= 2 and (x.is_cpu or (x.is_cuda and M <= 4))


def helion_backend_indicator(x: Tensor) -> bool:
    """The reference's Helion backend is not part of this build (always False)."""
    return False


class LTIMatrixRecurrence(Function):
    """Autograd Function of the native M x M LTI scan ``h[t] = A h[t-1] + x[t]``.

    A: ``[M, M]`` (shared) or ``[B, M, M]``; zi: ``[B, M]``; x: ``[B, T, M]``.
    backward: fused adjoint kernel without ``create_graph``, otherwise the
    composite formula through this Function (reference lti/ssm.py:67-96).
    jvp: one more scan with input ``dx + dA h[t-1]`` (lti/ssm.py:98-115).
    """

    @staticmethod
    def forward(A: Tensor, zi: Tensor, x: Tensor) -> Tensor:
        if x.size(-1) == 2:
            return torch.ops.philtorch.lti_recur2(A, zi, x)
        return torch.ops.philtorch.lti_recurN(A, zi, x)

    @staticmethod
    def setup_context(ctx: Any, inputs: tuple, output: Tensor) -> None:
        A, zi, _ = inputs
        ctx.save_for_backward(A, zi, output)
        ctx.save_for_forward(A, zi, output)

    @staticmethod
    def backward(ctx: Any, grad_y: Tensor):
        A, zi, y = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if not torch.is_grad_enabled():
            gA, gzi, gx = torch.ops.philtorch.lti_recurN_backward(A, zi, y, grad_y)
            return (gA if needs[0] else None, gzi if needs[1] else None, gx if needs[2] else None)
        AH = A.mT.conj_physical()
        lam = LTIMatrixRecurrence.apply(AH, torch.zeros_like(zi), grad_y.flip(1)).flip(1)
        grad_A = grad_zi = grad_x = None
        if needs[1]:
            grad_zi = (AH @ lam[:, 0, :, None]).squeeze(-1)
        if needs[2]:
            grad_x = lam
        if needs[0]:
            prev = torch.cat([zi.unsqueeze(1), y[:, :-1]], dim=1).conj_physical()
            per_row = lam.mT @ prev
            grad_A = per_row if A.dim() == 3 else per_row.sum(0)
        return grad_A, grad_zi, grad_x

    @staticmethod
    def jvp(ctx: Any, grad_A: Optional[Tensor], grad_zi: Optional[Tensor], grad_x: Optional[Tensor]) -> Tensor:
        A, zi, y = ctx.saved_tensors
        t_zi = grad_zi if grad_zi is not None else torch.zeros_like(zi)
        t_x = grad_x if grad_x is not None else torch.zeros_like(y)
        if grad_A is not None:
            prev = torch.cat([zi.unsqueeze(1), y[:, :-1]], dim=1)
            dA = grad_A if grad_A.dim() == 2 else grad_A.unsqueeze(-3)
            t_x = t_x + (dA @ prev.unsqueeze(-1)).squeeze(-1)
        return LTIMatrixRecurrence.apply(A, t_zi, t_x)


def _widen(x: Tensor, M: int) -> Tensor:
    return torch.cat([x.unsqueeze(-1), x.new_zeros(*x.shape, M - 1)], dim=-1)


def _recursion_loop(A: Tensor, zi: Tensor, x: Tensor, out_idx: Optional[int] = None) -> Tensor:
    """Per-step PyTorch loop (philtorch/lti/ssm.py:118-159)."""
    if x.dim() == 2:
        x = _widen(x, A.size(-1))
    h = zi
    outs = []
    for t in range(x.size(1)):
        h = (A @ h.unsqueeze(-1)).squeeze(-1) + x[:, t]
        outs.append(h if out_idx is None else h[:, out_idx])
    return torch.stack(outs, dim=1)


def _ext_ss_recur(A: Tensor, zi: Tensor, x: Tensor, *, out_idx: Optional[int] = None, **_) -> Tensor:
    """Native recursion (philtorch/lti/ssm.py:162-195)."""
    assert EXTENSION_LOADED or HELION_LOADED, "Compiled extension or the Helion backend is not available"
    if A.size(-1) == 1:
        xs = x if x.dim() == 2 else x.squeeze(-1)
        y = LTIRecurrence.apply(A[..., 0, 0], zi.squeeze(-1), xs).unsqueeze(-1)
    else:
        if x.dim() == 2:
            x = _widen(x, A.size(-1))
        y = LTIMatrixRecurrence.apply(A, zi, x)
    if out_idx is not None and y.dim() == 3:
        y = y[:, :, out_idx]
    return y


def state_space_recursion(
    A: Tensor, zi: Tensor, x: Tensor, *, unroll_factor: int = 1, out_idx: Optional[int] = None
) -> Tensor:
    """States of ``h[t] = A h[t-1] + x[t]`` (philtorch/lti/ssm.py:198-383).

    ``unroll_factor = 1`` runs the native scan: on the CPU for any order, on
    a HIP device for orders M <= 4 (the per-step PyTorch loop otherwise, or
    without the extension); ``k > 1`` a blocked PyTorch scan whose block
    gains are the powers ``A^1 .. A^k``.
    """
    assert x.dim() in (2, 3), f"Input signal must be 2D or 3D (batch, time, [features]), got {x.shape}"
    assert A.dim() in (2, 3), f"State matrix A must be 2D or 3D, got {A.shape}"
    assert A.size(-2) == A.size(-1), f"State matrix A must be square, got {A.shape}"
    if A.dim() == 3:
        assert x.size(0) == A.size(0), f"Batch size of A must match batch size of x, got A: {A.size(0)}, x: {x.size(0)}"
    if x.dim() == 3:
        assert A.size(-1) == x.size(-1), (
            f"Last dimension of A must match last dimension of x, got A: {A.size(-1)}, x: {x.size(-1)}"
        )
    batch, N = x.size(0), x.size(1)
    M = A.size(-1)
    assert zi.dim() == 2, f"Initial conditions zi must be 2D, got {zi.shape}"
    assert zi.size(0) == batch, f"Batch size of zi must match batch size of x, got zi: {zi.size(0)}, x: {batch}"
    assert zi.size(1) == M, f"Last dimension of zi must match last dimension of A, got zi: {zi.size(1)}, A: {M}"
    if unroll_factor < 1:
        raise ValueError("Unroll factor must be >= 1")
    k = unroll_factor
    if k == 1 or k >= N:
        if k == 1 and EXTENSION_LOADED and (x.is_cpu or (x.is_cuda and M <= 4)):
            return _ext_ss_recur(A, zi, x, out_idx=out_idx)
        return _recursion_loop(A, zi, x, out_idx=out_idx)

    if x.dim() == 2:
        x = _widen(x, M)
    pad = (-N) % k
    if pad:
        x = F.pad(x, (0, 0, 0, pad))
    xb = x.unflatten(1, (-1, k))  # [B, n, k, M]
    Ab = A if A.dim() == 2 else A.unsqueeze(1)  # broadcast over blocks
    h = torch.zeros_like(xb[:, :, 0])
    cols = []
    for i in range(k):
        h = (Ab @ h.unsqueeze(-1)).squeeze(-1) + xb[:, :, i]
        cols.append(h)
    local = torch.stack(cols, dim=2)
    powers = [A]
    for _ in range(k - 1):
        powers.append(A @ powers[-1])
    P = torch.stack(powers, dim=-3)  # [.., k, M, M]: A^1 .. A^k
    carries = state_space_recursion(P[..., -1, :, :], zi, local[:, :, -1], unroll_factor=k)
    prev = torch.cat([zi.unsqueeze(1), carries[:, :-1]], dim=1)  # [B, n, M]
    Pb = P if A.dim() == 2 else P.unsqueeze(1)
    out = local + (Pb @ prev.unsqueeze(2).unsqueeze(-1)).squeeze(-1)
    out = out.flatten(1, 2)[:, :N]
    return out if out_idx is None else out[..., out_idx]


def _ssm_C_D(h: Tensor, x: Tensor, C: Optional[Tensor], D: Optional[Tensor], batch_size: int, M: int) -> Tensor:
    """``y = C h + D x`` for the shapes of philtorch/lti/ssm.py:513-589."""
    features = -1 if x.dim() == 2 else x.size(-1)
    Dx = None
    if D is not None:
        shape = tuple(D.shape)
        if len(shape) == 1 and shape[0] == features:
            Dx = x @ D
        elif len(shape) == 1 and shape[0] == batch_size:
            assert x.dim() == 2, f"Input signal x must be 2D when D is of shape {batch_size,}, got {x.shape}"
            Dx = D.unsqueeze(1) * x
        elif shape in ((), (1,)):
            Dx = x * D
        elif len(shape) == 1:
            assert x.dim() == 2, f"Input signal x must be 2D when D is of shape (_,), got {x.shape}"
            Dx = D * x.unsqueeze(-1)
        elif len(shape) == 2 and shape == (batch_size, features):
            Dx = torch.linalg.vecdot(D.unsqueeze(1).conj(), x)
        elif len(shape) == 2 and shape[0] == batch_size:
            assert x.dim() == 2
            Dx = D.unsqueeze(1) * x.unsqueeze(-1)
        elif len(shape) == 2 and shape[1] == features:
            Dx = x @ D.T
        elif len(shape) == 3 and shape[0] == batch_size and shape[2] == features:
            Dx = torch.linalg.vecdot(D.unsqueeze(1).conj(), x.unsqueeze(-2))
        else:
            raise ValueError(f"Unsupported feedthrough matrix D of shape {D.shape}")
    if C is not None:
        shape = tuple(C.shape)
        if shape == (M,):
            Ch = h @ C
        elif len(shape) == 2 and shape == (batch_size, M):
            Ch = torch.linalg.vecdot(C.unsqueeze(1).conj(), h)
        elif len(shape) == 2 and shape[1] == M:
            Ch = h @ C.T
        elif len(shape) == 3 and shape[0] == batch_size and shape[2] == M:
            Ch = h @ C.mT
        else:
            raise ValueError(
                f"Output matrix C must be of shape ({M,}), ({batch_size, M}), (_, {M}), or ({batch_size}, _, {M}), got {C.shape}"
            )
    else:
        Ch = h
    return Ch + Dx if Dx is not None else Ch


def _fused_ss_applies(A: Tensor, x: Tensor, B, C, D, zi, unroll_factor, out_idx) -> bool:
    """A single-input single-output model of order <= 4 (2D x; B, C an
    M-vector per model or shared, or C replaced by out_idx; D one value per
    row or shared) on a HIP device with the native route requested
    (``unroll_factor=1``): philtorch::lti_ss runs B x, the scan, the state
    shift and C h + D x in one pass; gradients for x and zi are one pass of
    the adjoint model, and those of A, B, C, D two fused passes
    (philtorch::lti_ss_backward).  Forward-mode AD keeps the composed
    route."""
    from .. import EXTENSION_LOADED

    if not (EXTENSION_LOADED and x.is_cuda and unroll_factor == 1 and x.dim() == 2):
        return False
    if not hasattr(torch.ops.philtorch, "lti_ss"):
        return False
    batch, M = x.size(0), A.size(-1)
    if M > 4 or x.dtype not in (torch.float32, torch.float64):
        return False
    if any(t is not None and t.dtype != x.dtype for t in (A, B, C, D, zi)):
        return False
    if C is None and out_idx is None:
        return False

    def is_vec(t):
        return tuple(t.shape) in ((M,), (batch, M))

    if (B is not None and not is_vec(B)) or (C is not None and not is_vec(C)):
        return False
    if D is not None and not ((D.dim() <= 1 and D.numel() == 1) or tuple(D.shape) == (batch,)):
        return False
    import torch.autograd.forward_ad as fwad

    return all(t is None or fwad.unpack_dual(t).tangent is None for t in (A, B, C, D, zi, x))


def _mimo_operands(A: Tensor, x: Tensor, B, C, D, out_idx, batch: int, M: int):
    """The per-row matrices of philtorch::mimo_ss for a call of state_space,
    or None where the shapes fall outside it: ``(x3, Bm, Cm, Dm, vec)`` with
    x3 (batch, N, F), Bm (M, F) or (batch, M, F), Cm (P, M) or
    (batch, P, M), Dm None, (P, F) or (batch, P, F), and ``vec`` true where
    the reference's y is 2D (one output: C an M-vector or out_idx, D a
    feature vector or one value per row; y is then mimo_ss's squeezed).

    Each case mirrors a branch of the composed route (B:
    philtorch/lti/ssm.py:460-485; C and D: _ssm_C_D :513-589), tested in the
    same order, so the fused call reads every operand as the composed one
    does; B, C, D enter through views or products that autograd carries
    back to them.  A sum of a 2D and a 3D term (which the reference
    broadcasts) and shapes the composed route rejects stay with it."""
    two_d = x.dim() == 2
    Fn = 1 if two_d else x.size(-1)
    features = -1 if two_d else Fn
    eye = lambda n: torch.eye(n, dtype=x.dtype, device=x.device)  # noqa: E731
    if B is None:
        if two_d or Fn != M:
            return None
        Bm = eye(M)
    else:
        shape = tuple(B.shape)
        if shape == (M,):
            if not two_d:
                return None
            Bm = B.reshape(M, 1)
        elif len(shape) == 2 and shape == (batch, M) and two_d:
            Bm = B.reshape(batch, M, 1)
        elif len(shape) == 2 and shape == (M, features):
            Bm = B
        elif len(shape) == 3 and shape == (batch, M, features):
            Bm = B
        else:
            return None
    if C is None:
        if out_idx is None:
            Cm, c_vec = eye(M), False
        else:
            Cm, c_vec = eye(M)[out_idx].reshape(1, M), True
    else:
        shape = tuple(C.shape)
        if shape == (M,):
            Cm, c_vec = C.reshape(1, M), True
        elif len(shape) == 2 and shape == (batch, M):
            Cm, c_vec = C.reshape(batch, 1, M), True
        elif len(shape) == 2 and shape[1] == M:
            Cm, c_vec = C, False
        elif len(shape) == 3 and shape[0] == batch and shape[2] == M:
            Cm, c_vec = C, False
        else:
            return None
    Dm, d_vec = None, None
    if D is not None:
        shape = tuple(D.shape)
        if len(shape) == 1 and shape[0] == features:
            Dm, d_vec = D.reshape(1, Fn), True
        elif len(shape) == 1 and shape[0] == batch:
            if not two_d:
                return None
            Dm, d_vec = D.reshape(batch, 1, 1), True
        elif shape in ((), (1,)):
            if two_d:
                Dm, d_vec = D.reshape(1, 1), True
            else:
                Dm, d_vec = D.reshape(()) * eye(Fn), False
        elif len(shape) == 1:
            if not two_d:
                return None
            Dm, d_vec = D.reshape(shape[0], 1), False
        elif len(shape) == 2 and shape == (batch, features):
            Dm, d_vec = D.reshape(batch, 1, Fn), True
        elif len(shape) == 2 and shape[0] == batch:
            if not two_d:
                return None
            Dm, d_vec = D.reshape(batch, shape[1], 1), False
        elif len(shape) == 2 and shape[1] == features:
            Dm, d_vec = D, False
        elif len(shape) == 3 and shape[0] == batch and shape[2] == features:
            Dm, d_vec = D, False
        else:
            return None
        if d_vec != c_vec or Dm.size(-2) != Cm.size(-2):
            return None
    x3 = x.unsqueeze(-1) if two_d else x
    return x3, Bm, Cm, Dm, c_vec


def _mimo_applies(A: Tensor, x: Tensor, B, C, D, zi, unroll_factor) -> bool:
    """Whether a call outside the single-input single-output fused path can
    take philtorch::mimo_ss: order <= 4, float32 or float64 on a HIP device,
    the native route requested (``unroll_factor=1``), no forward-mode
    tangent (those keep the composed route); the widths are checked on the
    operands _mimo_operands builds."""
    from .. import EXTENSION_LOADED

    if not (EXTENSION_LOADED and x.is_cuda and unroll_factor == 1 and x.dim() in (2, 3)):
        return False
    if not hasattr(torch.ops.philtorch, "mimo_ss"):
        return False
    if A.size(-1) > 4 or x.dtype not in (torch.float32, torch.float64):
        return False
    if any(t is not None and t.dtype != x.dtype for t in (A, B, C, D, zi)):
        return False
    import torch.autograd.forward_ad as fwad

    return all(t is None or fwad.unpack_dual(t).tangent is None for t in (A, B, C, D, zi, x))


def _mimo_composite(A, Bm, Cm, Dm, zi, x, reverse=False):
    """(y, zf) of the composed route for philtorch::mimo_ss's operands (B x,
    the native scan, the shifted state sequence, C h + D x, in time-reversed
    order with ``reverse``): its autograd formula differentiates this under
    create_graph."""
    if reverse:
        y, zf = _mimo_composite(A, Bm, Cm, Dm, zi, x.flip(1))
        return y.flip(1), zf
    M = A.size(-1)
    zi = x.new_zeros(x.size(0), M) if zi is None else zi
    Bx = torch.matmul(x, Bm.mT)  # (batch, N, M)
    h = _ext_ss_recur(A, zi, Bx)
    zf = h[:, -1] if h.size(1) > 0 else zi
    h = torch.cat([zi.unsqueeze(1), h[:, :-1]], dim=1)
    y = torch.matmul(h, Cm.mT)
    if Dm is not None:
        y = y + torch.matmul(x, Dm.mT)
    return y, zf


def _state_space_composite(A, B, C, D, zi, x, out_idx=None):
    """(y, zf) of the composed route (B x, the native scan, the shifted state
    sequence, C h + D x) for what philtorch::lti_ss computes fused: its
    autograd formula differentiates this."""
    zi = x.new_zeros(x.size(0), A.size(-1)) if zi is None else zi
    return _state_space(A, x, B, C, D, zi, 1, None if C is not None else out_idx, fused=False)


def state_space(
    A: Tensor,
    x: Tensor,
    B: Optional[Tensor] = None,
    C: Optional[Tensor] = None,
    D: Optional[Tensor] = None,
    zi: Optional[Tensor] = None,
    unroll_factor: Optional[int] = None,
    out_idx: Optional[int] = None,
):
    """Outputs of ``h[t+1] = A h[t] + B x[t]``, ``y[t] = C h[t] + D x[t]``.

    Mirrors philtorch/lti/ssm.py:386-510; returns ``(y, zf)`` when ``zi`` is
    given.  ``unroll_factor=None`` means ``round(sqrt(N))`` (blocked PyTorch
    route) as in the reference; ``unroll_factor=1`` on a HIP device runs the
    native scan, a single-input single-output model of order <= 4 the fused
    philtorch::lti_ss, and other models of order <= 4 with at most four
    inputs and outputs per step (a 3D x, matrix-valued B, C, D) the fused
    philtorch::mimo_ss.
    """
    return _state_space(A, x, B, C, D, zi, unroll_factor, out_idx, fused=True)


def _state_space(A, x, B, C, D, zi, unroll_factor, out_idx, fused):
    assert x.dim() in (2, 3), f"Input signal must be 2D or 3D (batch, time, [features]), got {x.shape}"
    assert A.dim() in (2, 3), f"State matrix A must be 2D or 3D, got {A.shape}"
    assert A.size(-2) == A.size(-1), f"State matrix A must be square, got {A.shape}"
    if A.dim() == 3:
        assert x.size(0) == A.size(0), f"Batch size of A must match batch size of x, got A: {A.size(0)}, x: {x.size(0)}"
    if not (C is None or out_idx is None):
        raise ValueError("C and out_idx cannot be used together. Use either C or out_idx.")
    batch, N = x.size(0), x.size(1)
    M = A.size(-1)
    return_zf = zi is not None
    if zi is None:
        zi = x.new_zeros(batch, M)
    elif zi.dim() == 1:
        zi = zi.unsqueeze(0).expand(batch, -1)
    if unroll_factor is None:
        unroll_factor = round(N**0.5)
    if fused and _fused_ss_applies(A, x, B, C, D, zi, unroll_factor, out_idx):
        from .. import _has_op, _op_ctx

        # a coefficient with a gradient to come: the forward keeps its states
        # (lti_ss_states), which the coefficient backward would compute again
        keep = (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (A, B, C, D))
                and _has_op("lti_ss_states"))
        with _op_ctx(A, B, C, D, zi, x):
            args = (A, B, C, D, zi.contiguous() if return_zf else None, x, out_idx if C is None else 0)
            if keep:
                y, zf, _ = torch.ops.philtorch.lti_ss_states(*args)
            else:
                y, zf = torch.ops.philtorch.lti_ss(*args)
        return (y, zf) if return_zf else y
    ops = _mimo_operands(A, x, B, C, D, out_idx, batch, M) if fused and _mimo_applies(
        A, x, B, C, D, zi, unroll_factor) else None
    if ops is not None and ops[0].size(-1) <= 4 and ops[2].size(-2) <= 4:
        from .. import _op_ctx

        x3, Bm, Cm, Dm, vec = ops
        with _op_ctx(A, Bm, Cm, Dm, zi, x3):
            y, zf = torch.ops.philtorch.mimo_ss(A, Bm, Cm, Dm, zi.contiguous() if return_zf else None, x3)
        y = y.squeeze(-1) if vec else y
        return (y, zf) if return_zf else y
    features = -1 if x.dim() == 2 else x.size(-1)
    if B is not None:
        shape = tuple(B.shape)
        if shape == (M,):
            assert x.dim() == 2, f"Input signal x must be 2D when B is of shape {M,}, got {x.shape}"
            Bx = x.unsqueeze(-1) * B
        elif len(shape) == 2 and shape == (batch, M) and x.dim() == 2:
            Bx = x.unsqueeze(-1) * B.unsqueeze(1)
        elif len(shape) == 2 and shape == (M, features):
            Bx = x @ B.T
        elif len(shape) == 3 and shape == (batch, M, features):
            Bx = torch.linalg.vecdot(B.unsqueeze(1).conj(), x.unsqueeze(-2))
        else:
            raise ValueError(
                f"Input matrix B must be of shape ({M,}), ({batch, M}), ({M, features}), or ({batch, M, features}), got {B.shape}"
            )
    else:
        Bx = x

    native = extension_backend_indicator(x, M) and unroll_factor in (None, 1)
    runner = _ext_ss_recur if native else state_space_recursion
    if return_zf or out_idx is None:
        h = runner(A, zi, Bx, unroll_factor=unroll_factor, out_idx=None)
        zf = h[:, -1, :] if return_zf else None
        if out_idx is None:
            h = torch.cat([zi.unsqueeze(1), h[:, :-1]], dim=1)
        else:
            h = torch.cat([zi[:, None, out_idx], h[:, :-1, out_idx]], dim=1)
    else:
        zf = None
        h = runner(A, zi, Bx, unroll_factor=unroll_factor, out_idx=out_idx)
        h = torch.cat([zi[:, None, out_idx], h[:, :-1]], dim=1)
    y = _ssm_C_D(h, x, C, D, batch, M)
    return (y, zf) if return_zf else y


def diag_state_space(
    x: Tensor,
    L: Optional[Tensor] = None,
    V: Optional[Tensor] = None,
    Vinv: Optional[Tensor] = None,
    A: Optional[Tensor] = None,
    B: Optional[Tensor] = None,
    C: Optional[Tensor] = None,
    D: Optional[Tensor] = None,
    zi: Optional[Tensor] = None,
    out_idx: Optional[int] = None,
    unroll_factor: Optional[int] = None,
):
    """State-space model evaluated in the eigenbasis ``A = V diag(L) V^-1``.

    Mirrors philtorch/lti/ssm.py:592-833 for eigenvalues ``L`` given as a
    vector (with optional ``V``/``Vinv``) or a batch of vectors (with ``V`` or
    ``Vinv``), or a full ``A`` with ``L`` and ``V`` computed by
    ``torch.linalg.eig``.  The ``B*M`` independent scalar recursions run as
    one native ``lti_recur`` when ``unroll_factor`` is 1 and the input is on
    a HIP device.
    """
    assert x.dim() in (2, 3), f"Input signal must be 2D or 3D (batch, time, [features]), got {x.shape}"
    if not (C is None or out_idx is None):
        raise ValueError("C and out_idx cannot be used together. Use either C or out_idx.")
    batch, N = x.size(0), x.size(1)
    if unroll_factor is None:
        unroll_factor = round(N**0.5)
    if L is None:
        assert A is not None, "Either L or A must be provided"
        assert A.dim() in (2, 3), f"State matrix A must be 2D or 3D, got {A.shape}"
        L, V = torch.linalg.eig(A)
        Vinv = torch.linalg.inv(V)
        M = A.size(-1)
    else:
        if L.dim() == 1:
            M = L.size(0)
        elif L.dim() == 2 and L.size(0) == batch:
            M = L.size(1)
            assert not (V is None and Vinv is None), "P and Vinv cannot both be None when L is a batch of vectors"
        else:
            raise ValueError(f"L must be a vector or a batch of vectors, got {L.shape}")
        if V is None and Vinv is None:
            V = Vinv = torch.eye(M, device=x.device, dtype=x.dtype)
        elif V is None:
            V = torch.linalg.inv(Vinv)
        elif Vinv is None:
            Vinv = torch.linalg.inv(V)

    return_zf = zi is not None
    if zi is None:
        zi = x.new_zeros(batch, M)
    elif zi.dim() == 1:
        zi = zi.unsqueeze(0).expand(batch, -1)

    x_orig = x
    if Vinv.is_complex():
        if not zi.is_complex():
            zi = zi + 0j
        if not x.is_complex():
            x = x + 0j
        if B is not None and not B.is_complex():
            B = B + 0j
    Vinv_zi = zi @ Vinv.T if Vinv.dim() == 2 else torch.linalg.vecdot(Vinv.conj(), zi.unsqueeze(1))
    features = -1 if x.dim() == 2 else x.size(-1)
    if B is not None:
        shape = tuple(B.shape)
        if shape == (M,):
            VB = Vinv @ B
            VBx = x.unsqueeze(-1) * (VB.unsqueeze(1) if VB.dim() == 2 else VB)
        elif len(shape) == 2 and shape == (batch, M):
            VB = B @ Vinv.T if Vinv.dim() == 2 else torch.linalg.vecdot(Vinv.conj(), B.unsqueeze(1))
            VBx = x.unsqueeze(-1) * VB.unsqueeze(1)
        elif len(shape) == 2 and shape == (M, features):
            VBx = x @ (Vinv @ B).mT
        elif len(shape) == 3 and shape == (batch, M, features):
            VBx = torch.linalg.vecdot((Vinv @ B).unsqueeze(1).conj(), x.unsqueeze(-2))
        else:
            raise ValueError(f"Unsupported input matrix B of shape {B.shape}")
    elif x.dim() == 2:
        VBx = x.unsqueeze(-1) * (Vinv[:, 0] if Vinv.dim() == 2 else Vinv[:, None, :, 0])
    else:
        VBx = x @ Vinv.mT

    native = EXTENSION_LOADED and (x.is_cpu or x.is_cuda) and unroll_factor in (None, 1)
    runner = LTIRecurrence.apply if native else partial(linear_recurrence, unroll_factor=unroll_factor)
    coef = L.broadcast_to((batch, M)).flatten(0, 1)
    if native:
        coef = coef.to(VBx.dtype)
    Vinv_h = runner(coef, Vinv_zi.flatten().to(VBx.dtype), VBx.mT.flatten(0, 1)).unflatten(0, (batch, M))
    if not return_zf and out_idx is not None:
        h = torch.cat([zi[:, None, out_idx], (V[..., out_idx, None, :] @ Vinv_h[..., :-1]).squeeze(-2)], dim=1)
        zf = None
    else:
        h = (V @ Vinv_h).mT
        zf = h[:, -1, :] if return_zf else None
        if out_idx is None:
            h = torch.cat([zi.unsqueeze(1), h[:, :-1]], dim=1)
        else:
            h = torch.cat([zi[:, None, out_idx], h[:, :-1, out_idx]], dim=1)
    if C is not None and not C.is_complex():
        h = h.real
        zf = zf.real if return_zf else None
    y = _ssm_C_D(h, x_orig, C, D, batch, M)
    return (y, zf) if return_zf else y
