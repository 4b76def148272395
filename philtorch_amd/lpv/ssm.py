"""Time-varying (LPV) state-space recursion and models (philtorch/lpv/ssm.py).

``MatrixRecurrence`` is the autograd Function over ``philtorch::recur2`` /
``philtorch::recurN`` (reference philtorch/lpv/ssm.py:34-115).  On a HIP
device with ``unroll_factor == 1`` the recursion runs as one native scan;
elsewhere the reference's pure-PyTorch routes are kept: a per-step loop, or a
two-level blocked scan for ``unroll_factor > 1``.

The M = 1 case of ``_ext_ss_recur`` calls the native scalar scan
``philtorch::recur``; the reference sends it to the third-party
``torchlpc.sample_wise_lpc`` (philtorch/lpv/ssm.py:188-195), which computes
the same recurrence with the coefficient negated.
"""
from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.autograd import Function

from .. import EXTENSION_LOADED, HELION_LOADED


def extension_backend_indicator(x: Tensor, M: int) -> bool:
    """True when the native scan serves this input: extension loaded, and
    the tensor on the CPU (any order) or on a HIP device with a state of
    order M <= 4 (the reference, philtorch/lpv/ssm.py:20-26, takes the CPU
    for any order and the GPU for M <= 2)."""
    return EXTENSION_LOADED and (x.is_cpu or (x.is_cuda and M <= 4))


class MatrixRecurrence(Function):
    """Autograd Function of the native M x M LPV scan ``h[t] = A[t] h[t-1] + x[t]``.

    A: ``[T, M, M]`` (shared) or ``[B, T, M, M]``; zi: ``[B, M]``; x: ``[B, T, M]``.
    backward: fused adjoint kernel without ``create_graph``, otherwise the
    composite formula through this Function (reference lpv/ssm.py:64-99).
    jvp: one more scan with input ``dx + dA h[t-1]`` (lpv/ssm.py:101-115).
    """

    @staticmethod
    def forward(A: Tensor, zi: Tensor, x: Tensor) -> Tensor:
        if x.size(-1) == 2:
            return torch.ops.philtorch.recur2(A, zi, x)
        return torch.ops.philtorch.recurN(A, zi, x)

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
            gA, gzi, gx = torch.ops.philtorch.recurN_backward(A, zi, y, grad_y)
            return (gA if needs[0] else None, gzi if needs[1] else None, gx if needs[2] else None)
        AH = A.mT.conj_physical()
        coef = torch.roll(AH, -1, dims=-3).flip(-3)
        lam = MatrixRecurrence.apply(coef, torch.zeros_like(zi), grad_y.flip(1)).flip(1)
        grad_A = grad_zi = grad_x = None
        if needs[1]:
            grad_zi = (AH[..., 0, :, :] @ lam[:, 0, :, None]).squeeze(-1)
        if needs[2]:
            grad_x = lam
        if needs[0]:
            prev = torch.cat([zi.unsqueeze(1), y[:, :-1]], dim=1).conj_physical()
            per_step = lam.unsqueeze(-1) * prev.unsqueeze(-2)
            grad_A = per_step if A.dim() == 4 else per_step.sum(0)
        return grad_A, grad_zi, grad_x

    @staticmethod
    def jvp(ctx: Any, grad_A: Optional[Tensor], grad_zi: Optional[Tensor], grad_x: Optional[Tensor]) -> Tensor:
        A, zi, y = ctx.saved_tensors
        t_zi = grad_zi if grad_zi is not None else torch.zeros_like(zi)
        t_x = grad_x if grad_x is not None else torch.zeros_like(y)
        if grad_A is not None:
            prev = torch.cat([zi.unsqueeze(1), y[:, :-1]], dim=1)
            t_x = t_x + (grad_A @ prev.unsqueeze(-1)).squeeze(-1)
        return MatrixRecurrence.apply(A, t_zi, t_x)


def _widen(x: Tensor, M: int) -> Tensor:
    """``[B, T]`` input driving the first state only -> ``[B, T, M]``."""
    return torch.cat([x.unsqueeze(-1), x.new_zeros(*x.shape, M - 1)], dim=-1)


def _recursion_loop(A: Tensor, zi: Tensor, x: Tensor, out_idx: Optional[int] = None) -> Tensor:
    """Per-step PyTorch loop (philtorch/lpv/ssm.py:118-164)."""
    assert x.size(1) == A.size(-3), (
        f"State matrix A must have the same time dimension as x, got A: {A.size(-3)}, x: {x.size(1)}"
    )
    if x.dim() == 2:
        x = _widen(x, A.size(-1))
    h = zi
    outs = []
    for t in range(x.size(1)):
        At = A[t] if A.dim() == 3 else A[:, t]
        h = (At @ h.unsqueeze(-1)).squeeze(-1) + x[:, t]
        outs.append(h if out_idx is None else h[:, out_idx])
    return torch.stack(outs, dim=1)


def _ext_ss_recur(A: Tensor, zi: Tensor, x: Tensor, *, out_idx: Optional[int] = None, **_) -> Tensor:
    """Native recursion (philtorch/lpv/ssm.py:167-205)."""
    assert EXTENSION_LOADED or HELION_LOADED, "Compiled extension or the Helion backend is not available"
    M = A.size(-1)
    if M == 1:
        xs = x if x.dim() == 2 else x.squeeze(-1)
        coef = A[..., 0, 0]  # [T] shared or [B, T]
        y = torch.ops.philtorch.recur(coef, zi.reshape(-1), xs).unsqueeze(-1)
    else:
        if x.dim() == 2:
            x = _widen(x, M)
        y = MatrixRecurrence.apply(A, zi, x)
    if out_idx is not None and y.dim() == 3:
        y = y[:, :, out_idx]
    return y


def _prefix_products(A: Tensor) -> Tensor:
    """P[..., i, :, :] = A[i] ... A[1] A[0] along dim -3."""
    out = [A[..., 0, :, :]]
    for i in range(1, A.size(-3)):
        out.append(A[..., i, :, :] @ out[-1])
    return torch.stack(out, dim=-3)


def state_space_recursion(
    A: Tensor, zi: Tensor, x: Tensor, *, unroll_factor: int = 1, out_idx: Optional[int] = None
) -> Tensor:
    """States of ``h[t] = A[t] h[t-1] + x[t]`` (philtorch/lpv/ssm.py:208-334).

    Args:
        A: ``[N, M, M]`` or ``[B, N, M, M]``.
        zi: ``[B, M]`` initial states.
        x: ``[B, N, M]`` or ``[B, N]`` (drives the first state).
        unroll_factor: 1 = the native scan where the backend indicator
            allows it (CPU tensors of any order, HIP tensors of order <= 4;
            the per-step PyTorch loop otherwise); ``k > 1`` = blocked PyTorch
            scan with blocks of ``k`` steps.
        out_idx: return only this state index.
    Returns:
        ``[B, N, M]`` (or ``[B, N]`` with ``out_idx``).
    """
    assert x.dim() in (2, 3), f"Input signal must be 2D or 3D (batch, time, [features]), got {x.shape}"
    assert A.dim() in (3, 4), f"State matrix A must be 3D or 4D, got {A.shape}"
    assert A.size(-2) == A.size(-1), f"State matrix A must be square, got {A.shape}"
    assert A.size(-3) == x.size(1), (
        f"State matrix A must have the same time dimension as x, got A: {A.size(-3)}, x: {x.size(1)}"
    )
    if A.dim() == 4:
        assert x.size(0) == A.size(0), (
            f"Batch size of A must match batch size of x, got A: {A.size(0)}, x: {x.size(0)}"
        )
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
        if k == 1 and extension_backend_indicator(x, M):
            return _ext_ss_recur(A, zi, x, out_idx=out_idx)
        return _recursion_loop(A, zi, x, out_idx=out_idx)

    if x.dim() == 2:
        x = _widen(x, M)
    pad = (-N) % k
    if pad:
        x = F.pad(x, (0, 0, 0, pad))
        A = F.pad(A, (0, 0, 0, 0, 0, pad))
    xb = x.unflatten(1, (-1, k))  # [B, n, k, M]
    Ab = A.unflatten(-3, (-1, k))  # [n, k, M, M] or [B, n, k, M, M]
    # block-local scans from a zero state, k vectorised steps
    h = torch.zeros_like(xb[:, :, 0])
    cols = []
    for i in range(k):
        h = (Ab[..., i, :, :] @ h.unsqueeze(-1)).squeeze(-1) + xb[:, :, i]
        cols.append(h)
    local = torch.stack(cols, dim=2)  # [B, n, k, M]
    gains = _prefix_products(Ab)  # [.., n, k, M, M]
    carries = state_space_recursion(gains[..., -1, :, :], zi, local[:, :, -1], unroll_factor=k)  # [B, n, M]
    prev = torch.cat([zi.unsqueeze(1), carries[:, :-1]], dim=1)  # state entering each block
    out = local + (gains @ prev.unsqueeze(2).unsqueeze(-1)).squeeze(-1)
    out = out.flatten(1, 2)[:, :N]
    return out if out_idx is None else out[..., out_idx]


def _apply_B(x: Tensor, B: Optional[Tensor], batch: int, N: int, M: int, features: int) -> Tensor:
    """Input matrix shapes of philtorch/lpv/ssm.py:413-454."""
    if B is None:
        return x
    shape = tuple(B.shape)
    if shape == (M,):
        assert x.dim() == 2, f"Input signal x must be 2D when B is of shape {M,}, got {x.shape}"
        return x.unsqueeze(-1) * B
    if len(shape) == 2 and shape == (M, features):
        return x @ B.T
    if len(shape) == 2 and shape == (N, M):
        assert x.dim() == 2
        return x.unsqueeze(-1) * B
    if len(shape) == 2 and shape == (batch, M):
        assert x.dim() == 2
        return x.unsqueeze(-1) * B.unsqueeze(1)
    if len(shape) == 3 and shape == (N, M, features):
        return torch.linalg.vecdot(B.conj(), x.unsqueeze(-2))
    if len(shape) == 3 and shape == (batch, N, M):
        assert x.dim() == 2
        return x.unsqueeze(-1) * B
    if len(shape) == 3 and shape == (batch, M, features):
        return torch.linalg.vecdot(B.unsqueeze(1).conj(), x.unsqueeze(-2))
    if len(shape) == 4 and shape == (batch, N, M, features):
        return torch.linalg.vecdot(B.conj(), x.unsqueeze(-2))
    raise ValueError(
        f"Input matrix B must be of shape ({M},), ({M, features}), ({N, M}), ({batch, M}), "
        f"({N, M, features}), ({batch, N, M}), ({batch, M, features}), or ({batch, N, M, features}), got {B.shape}"
    )


def _apply_D(x: Tensor, D: Optional[Tensor], batch: int, N: int, features: int) -> Optional[Tensor]:
    """Feedthrough shapes (the common subset of philtorch/lpv/ssm.py:480-547)."""
    if D is None:
        return None
    shape = tuple(D.shape)
    if shape in ((), (1,)):
        return x * D
    if len(shape) == 1:
        if shape[0] == features:
            return x @ D
        if shape[0] == N and x.dim() == 2:
            return D * x
        if shape[0] == batch and x.dim() == 2:
            return D.unsqueeze(1) * x
        assert x.dim() == 2, f"Input signal x must be 2D when D is of shape {D.shape}, got {x.shape}"
        return x.unsqueeze(-1) * D
    if len(shape) == 2:
        # the reference's case order: (N, F), (batch, F), (N, _), (batch, N),
        # (batch, _), (_, F); so (N, _) wins over (batch, N) when batch == N
        if shape == (N, features):
            return torch.linalg.vecdot(D.conj(), x)
        if shape == (batch, features):
            return torch.linalg.vecdot(D.conj().unsqueeze(1), x)
        if shape[0] == N:
            assert x.dim() == 2, f"Input signal x must be 2D when D is of shape ({N, features}), got {x.shape}"
            return D * x.unsqueeze(-1)
        if shape == (batch, N) and x.dim() == 2:
            return D * x
        if shape[0] == batch and x.dim() == 2:
            return D.unsqueeze(1) * x.unsqueeze(-1)
        if shape[1] == features:
            return x @ D.T
    if len(shape) == 3:
        if shape == (batch, N, features):
            return torch.linalg.vecdot(D.conj(), x)
        if shape[0] == batch and shape[2] == features:
            return x @ D.mT
        if shape[0] == N and shape[2] == features:
            return torch.linalg.vecdot(D.conj(), x.unsqueeze(-2))
        if shape[:2] == (batch, N) and x.dim() == 2:
            return D * x.unsqueeze(-1)
    if len(shape) == 4 and shape[0] == batch and shape[1] == N and shape[3] == features:
        return torch.linalg.vecdot(D.conj(), x.unsqueeze(-2))
    raise ValueError(f"Unsupported feedthrough matrix D of shape {D.shape}")


def _apply_C(h: Tensor, C: Optional[Tensor], batch: int, N: int, M: int) -> Tensor:
    """Output matrix shapes of philtorch/lpv/ssm.py:549-573."""
    if C is None:
        return h
    shape = tuple(C.shape)
    if shape == (M,):
        return h @ C
    if len(shape) == 2 and shape == (N, M):
        return torch.linalg.vecdot(C.conj(), h)
    if len(shape) == 2 and shape == (batch, M):
        return torch.linalg.vecdot(C.unsqueeze(1).conj(), h)
    if len(shape) == 2 and shape[1] == M:
        return h @ C.T
    if len(shape) == 3 and shape[0] == N and shape[2] == M:
        return torch.linalg.vecdot(C.conj(), h.unsqueeze(-2))
    if len(shape) == 3 and shape == (batch, N, M):
        return torch.linalg.vecdot(C.conj(), h)
    if len(shape) == 3 and shape[0] == batch and shape[2] == M:
        return h @ C.mT
    if len(shape) == 4 and shape[0] == batch and shape[1] == N and shape[3] == M:
        return torch.linalg.vecdot(C.conj(), h.unsqueeze(-2))
    raise ValueError(
        f"Output matrix C must be of shape ({M,}), ({N, M}), ({batch, M}), ({batch, N, M}), or ({batch, N, '_', M}), "
        f"got {C.shape}"
    )


def _lpv_siso_operands(x: Tensor, B, C, D, out_idx, batch: int, N: int, M: int):
    """B, C as (1 | batch, 1 | N, M) and D as (1 | batch, 1 | N) views when the
    model has one input and one output, following the shape cases of
    philtorch/lpv/ssm.py:413-454 (B), :480-547 (D) and :549-573 (C) in their
    order; None when it has not (a state or multi-output y, features)."""
    if x.dim() != 2:
        return None
    if B is not None:
        s = tuple(B.shape)
        if s == (M,):
            B = B.reshape(1, 1, M)
        elif s == (N, M):
            B = B.reshape(1, N, M)
        elif s == (batch, M):
            B = B.reshape(batch, 1, M)
        elif s == (batch, N, M):
            pass
        else:
            return None
    if C is None:
        if out_idx is None:
            return None
    else:
        s = tuple(C.shape)
        if s == (M,):
            C = C.reshape(1, 1, M)
        elif s == (N, M):
            C = C.reshape(1, N, M)
        elif s == (batch, M):
            C = C.reshape(batch, 1, M)
        elif len(s) == 3 and s[0] != N and s == (batch, N, M):
            pass
        else:
            return None
    if D is not None:
        s = tuple(D.shape)
        if s in ((), (1,)):
            D = D.reshape(1, 1)
        elif len(s) == 1 and s[0] == N:
            D = D.reshape(1, N)
        elif len(s) == 1 and s[0] == batch:
            D = D.reshape(batch, 1)
        elif len(s) == 2 and s[0] != N and s == (batch, N):
            pass
        else:
            return None
    return B, C, D


def _lpv_state_space_composite(A, B, C, D, zi, x, out_idx=0):
    """The route philtorch::lpv_ss replaces, on canonical operands (B, C as
    (1 | batch, 1 | N, M), D as (1 | batch, 1 | N)): B x, the native LPV
    scan, the state shift, C h + D x; returns (y, zf).  Differentiable."""
    batch, N = x.shape
    M = A.size(-1)
    z = zi if zi is not None else x.new_zeros(batch, M)
    Bx = x.unsqueeze(-1) * B if B is not None else _widen(x, M)
    h = _ext_ss_recur(A, z, Bx)
    zf = h[:, -1] if N > 0 else z
    hp = torch.cat([z.unsqueeze(1), h[:, :-1]], dim=1)
    y = (hp * C).sum(-1) if C is not None else hp[..., out_idx]
    if D is not None:
        y = y + D * x
    return y, zf


def _lpv_mimo_operands(x: Tensor, B, C, D, out_idx, batch: int, N: int, M: int):
    """The per-row (or shared) matrices of philtorch::lpv_mimo_ss for a call
    of state_space whose B, C, D are constant in time, or None where they
    are not or the shapes fall outside it: ``(x3, Bm, Cm, Dm, vec)`` with x3
    (batch, N, F), Bm (M, F) or (batch, M, F), Cm (P, M) or (batch, P, M),
    Dm None, (P, F) or (batch, P, F), and ``vec`` true where the
    reference's y is 2D (one output).  Each case mirrors a branch of the
    composed route (_apply_B: philtorch/lpv/ssm.py:413-454; _apply_D
    :480-547; _apply_C :549-573), tested in the same order, so a shape is
    read as the composed route reads it; a branch whose operand varies along
    time (an N axis) returns None, as does a one-output term added to a
    multi-output one (which the reference broadcasts)."""
    two_d = x.dim() == 2
    Fn = 1 if two_d else x.size(-1)
    features = -1 if two_d else Fn
    eye = lambda n: torch.eye(n, dtype=x.dtype, device=x.device)  # noqa: E731
    if B is None:
        if two_d or Fn != M:
            return None
        Bm = eye(M)
    else:
        s = tuple(B.shape)
        if s == (M,):
            if not two_d:
                return None
            Bm = B.reshape(M, 1)
        elif len(s) == 2 and s == (M, features):
            Bm = B
        elif len(s) == 2 and s == (N, M):
            return None
        elif len(s) == 2 and s == (batch, M):
            if not two_d:
                return None
            Bm = B.reshape(batch, M, 1)
        elif len(s) == 3 and s == (N, M, features):
            return None
        elif len(s) == 3 and s == (batch, N, M):
            return None
        elif len(s) == 3 and s == (batch, M, features):
            Bm = B
        else:
            return None
    if C is None:
        if out_idx is None:
            Cm, c_vec = eye(M), False
        else:
            Cm, c_vec = eye(M)[out_idx].reshape(1, M), True
    else:
        s = tuple(C.shape)
        if s == (M,):
            Cm, c_vec = C.reshape(1, M), True
        elif len(s) == 2 and s == (N, M):
            return None
        elif len(s) == 2 and s == (batch, M):
            Cm, c_vec = C.reshape(batch, 1, M), True
        elif len(s) == 2 and s[1] == M:
            Cm, c_vec = C, False
        elif len(s) == 3 and s[0] == N and s[2] == M:
            return None
        elif len(s) == 3 and s == (batch, N, M):
            return None
        elif len(s) == 3 and s[0] == batch and s[2] == M:
            Cm, c_vec = C, False
        else:
            return None
    Dm, d_vec = None, None
    if D is not None:
        s = tuple(D.shape)
        if s in ((), (1,)):
            if two_d:
                Dm, d_vec = D.reshape(1, 1), True
            else:
                Dm, d_vec = D.reshape(()) * eye(Fn), False
        elif len(s) == 1:
            if s[0] == features:
                Dm, d_vec = D.reshape(1, Fn), True
            elif not two_d or s[0] == N:
                return None
            elif s[0] == batch:
                Dm, d_vec = D.reshape(batch, 1, 1), True
            else:
                Dm, d_vec = D.reshape(s[0], 1), False
        elif len(s) == 2:
            if s == (N, features):
                return None
            if s == (batch, features):
                Dm, d_vec = D.reshape(batch, 1, Fn), True
            elif s[0] == N or (s == (batch, N) and two_d):
                return None
            elif s[0] == batch and two_d:
                Dm, d_vec = D.reshape(batch, s[1], 1), False
            elif s[1] == features:
                Dm, d_vec = D, False
            else:
                return None
        elif len(s) == 3:
            if s == (batch, N, features):
                return None
            if s[0] == batch and s[2] == features:
                Dm, d_vec = D, False
            else:
                return None
        else:
            return None
        if d_vec != c_vec or Dm.size(-2) != Cm.size(-2):
            return None
    return (x.unsqueeze(-1) if two_d else x), Bm, Cm, Dm, c_vec


def _lpv_mimo_applies(A: Tensor, x: Tensor, zi: Optional[Tensor], ops, native: bool) -> bool:
    """Whether _lpv_mimo_operands' matrices run philtorch::lpv_mimo_ss:
    order <= 4, at most four inputs and outputs per step, float32 or float64
    on a HIP device with the native route requested, no forward-mode
    tangent."""
    from .. import EXTENSION_LOADED

    if not (native and EXTENSION_LOADED and x.is_cuda and ops is not None and hasattr(torch.ops.philtorch, "lpv_mimo_ss")):
        return False
    x3, Bm, Cm, Dm, _ = ops
    if x.dtype not in (torch.float32, torch.float64) or A.size(-1) > 4 or x3.size(-1) > 4 or Cm.size(-2) > 4:
        return False
    tensors = [A, x, Bm, Cm] + [t for t in (Dm, zi) if t is not None]
    if any(t.dtype != x.dtype or t.device != x.device for t in tensors):
        return False
    if A.dim() == 4 and A.size(0) != x.size(0):
        return False
    import torch.autograd.forward_ad as fwad

    return all(fwad.unpack_dual(t).tangent is None for t in tensors)


def _lpv_mimo_composite(A, Bm, Cm, Dm, zi, x, reverse=False, transpose_A=False):
    """(y, zf) of the composed route for philtorch::lpv_mimo_ss's operands (B
    x, the native LPV scan, the shifted state sequence, C h + D x; A[t]^T
    with ``transpose_A``, in time-reversed order with ``reverse``): its
    autograd formula differentiates this under create_graph."""
    if transpose_A:
        A = A.mT
    if reverse:
        y, zf = _lpv_mimo_composite(A.flip(-3), Bm, Cm, Dm, zi, x.flip(1))
        return y.flip(1), zf
    M = A.size(-1)
    zi = x.new_zeros(x.size(0), M) if zi is None else zi
    Bx = torch.matmul(x, Bm.mT)  # (batch, N, M)
    h = _ext_ss_recur(A.contiguous(), zi, Bx)
    zf = h[:, -1] if h.size(1) > 0 else zi
    h = torch.cat([zi.unsqueeze(1), h[:, :-1]], dim=1)
    y = torch.matmul(h, Cm.mT)
    if Dm is not None:
        y = y + torch.matmul(x, Dm.mT)
    return y, zf


# Above this many bytes of per-row, per-step gradients of the operands that
# the rows share but that vary along time (A (T, M, M); B, C, D with one row
# and T steps), which philtorch::lpv_ss_backward writes for every row before
# it sums them, the coefficient gradients take the composed route's autograd
# instead, which reduces over the rows as it goes (the reference's
# algorithm, philtorch/lpv/ssm.py:337-581).  At B = 32, T = 2^20, M = 4 fp32
# the scratch for A alone is 2 GiB.
_LPV_ROW_SCRATCH_LIMIT = 512 << 20


def _lpv_row_scratch_bytes(A: Tensor, B, C, D, x: Tensor, needs) -> int:
    """Bytes of per-row step gradients philtorch::lpv_ss_backward would
    write for operands shared by the rows and varying along time, for the
    gradients `needs` asks for (A, B, C, D order)."""
    batch, T = x.shape
    M = A.size(-1)
    per_step = 0
    if needs[0] and A.dim() == 3:
        per_step += M * M
    for t, width, need in ((B, M, needs[1]), (C, M, needs[2]), (D, 1, needs[3])):
        if need and t is not None and (t.size(0) == 1 or t.stride(0) == 0) and t.size(1) > 1 and t.stride(1) != 0:
            per_step += width
    return batch * T * per_step * x.element_size()


def _fused_lpv_ss_applies(A: Tensor, x: Tensor, zi: Optional[Tensor], ops, native: bool) -> bool:
    """A model of order <= 4 with one input and one output on a HIP device,
    the native route requested and no tangent: philtorch::lpv_ss runs it in
    one pass; gradients w.r.t. x and zi are one more pass of its adjoint,
    those of A, B, C, D two fused passes (philtorch::lpv_ss_backward)."""
    from .. import EXTENSION_LOADED

    if not (native and EXTENSION_LOADED and x.is_cuda and ops is not None and hasattr(torch.ops.philtorch, "lpv_ss")):
        return False
    if x.dtype not in (torch.float32, torch.float64) or A.size(-1) > 4:
        return False
    tensors = [A, x] + [t for t in (zi, *ops) if t is not None]
    if any(t.dtype != x.dtype or t.device != x.device for t in tensors):
        return False
    if A.dim() == 4 and A.size(0) != x.size(0):
        return False
    import torch.autograd.forward_ad as fwad

    return all(fwad.unpack_dual(t).tangent is None for t in tensors)


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
    """Outputs of ``h[t+1] = A[t] h[t] + B x[t]``, ``y[t] = C h[t] + D x[t]``.

    Mirrors philtorch/lpv/ssm.py:337-581: when ``zi`` is given, returns
    ``(y, zf)``.  ``unroll_factor=None`` means ``round(sqrt(N))`` (the
    blocked PyTorch route); ``unroll_factor=1`` on a HIP device runs the
    native scan.  A model of order <= 4 with one input and one output (2D x;
    B, C per row and/or per step or absent / out_idx; D per row and/or per
    step) runs philtorch::lpv_ss: B x, the scan, the state shift and
    C h + D x in one pass; its adjoint gives the gradients w.r.t. x and zi,
    and philtorch::lpv_ss_backward those of A, B, C, D.  A model with up to
    four inputs and outputs per step (3D x, matrix-valued B, C, D) whose B,
    C, D are constant in time runs philtorch::lpv_mimo_ss the same way.
    """
    assert x.dim() in (2, 3), f"Input signal must be 2D or 3D (batch, time, [features]), got {x.shape}"
    assert A.dim() in (3, 4), f"State matrix A must be 3D or 4D, got {A.shape}"
    assert A.size(-2) == A.size(-1), f"State matrix A must be square, got {A.shape}"
    assert A.size(-3) == x.size(1), (
        f"State matrix A must have the same time dimension as x, got A: {A.size(-3)}, x: {x.size(1)}"
    )
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
    features = -1 if x.dim() == 2 else x.size(-1)
    native = extension_backend_indicator(x, M) and unroll_factor in (None, 1)
    ops = _lpv_siso_operands(x, B, C, D, out_idx, batch, N, M)
    if _fused_lpv_ss_applies(A, x, zi if return_zf else None, ops, native):
        from .. import _has_op, _op_ctx

        # a coefficient with a gradient to come: the forward keeps its states
        # (lpv_ss_states), which the coefficient backward would compute again
        keep = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (A, *ops))
        with _op_ctx(A, *ops, zi, x):
            args = (A, ops[0], ops[1], ops[2], zi.contiguous() if return_zf else None, x,
                    0 if out_idx is None else out_idx)
            if keep and _has_op("lpv_ss_states"):
                y, zf, _ = torch.ops.philtorch.lpv_ss_states(*args)
            else:
                y, zf = torch.ops.philtorch.lpv_ss(*args)
        return (y, zf) if return_zf else y
    mops = _lpv_mimo_operands(x, B, C, D, out_idx, batch, N, M) if native else None
    if _lpv_mimo_applies(A, x, zi if return_zf else None, mops, native):
        from .. import _has_op, _op_ctx

        x3, Bm, Cm, Dm, vec = mops
        # a coefficient with a gradient to come: the forward keeps its states
        # (lpv_mimo_ss_states, where outputs and states fit four planes)
        keep = (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (A, Bm, Cm, Dm))
                and Cm.size(-2) + M <= 4 and _has_op("lpv_mimo_ss_states"))
        with _op_ctx(A, Bm, Cm, Dm, zi, x3):
            args = (A, Bm, Cm, Dm, zi.contiguous() if return_zf else None, x3)
            if keep:
                y, zf, _ = torch.ops.philtorch.lpv_mimo_ss_states(*args)
            else:
                y, zf = torch.ops.philtorch.lpv_mimo_ss(*args)
        y = y.squeeze(-1) if vec else y
        return (y, zf) if return_zf else y
    Bx = _apply_B(x, B, batch, N, M, features)

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

    Dx = _apply_D(x, D, batch, N, features)
    y = _apply_C(h, C, batch, N, M)
    if Dx is not None:
        y = y + Dx
    return (y, zf) if return_zf else y
