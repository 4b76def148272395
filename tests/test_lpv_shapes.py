"""CPU checks of the LPV state-space shape handling: which B, C, D shapes
make a single-output model for the fused route (philtorch::lpv_ss), read in
the reference's case order (philtorch/lpv/ssm.py:413-454 for B, :480-547
for D, :549-573 for C), including the ambiguous shapes where the batch size
equals the number of steps."""
import torch

from philtorch_amd.lpv import ssm


def _ops(batch, N, M, B=None, C=None, D=None, out_idx=None):
    x = torch.zeros(batch, N)
    return ssm._lpv_siso_operands(x, B, C, D, out_idx, batch, N, M)


def test_siso_operand_layouts():
    batch, N, M = 3, 5, 2
    B, C, D = _ops(batch, N, M, B=torch.ones(M), C=torch.ones(N, M), D=torch.ones(batch, N))
    assert B.shape == (1, 1, M) and C.shape == (1, N, M) and D.shape == (batch, N)
    B, C, D = _ops(batch, N, M, B=torch.ones(batch, M), C=torch.ones(batch, N, M), D=torch.ones(()))
    assert B.shape == (batch, 1, M) and C.shape == (batch, N, M) and D.shape == (1, 1)
    B, C, D = _ops(batch, N, M, B=torch.ones(batch, N, M), out_idx=1, D=torch.ones(N))
    assert B.shape == (batch, N, M) and C is None and D.shape == (1, N)
    assert _ops(batch, N, M, D=torch.ones(batch), out_idx=0)[2].shape == (batch, 1)


def test_multi_output_shapes_are_not_fused():
    batch, N, M = 3, 5, 2
    assert _ops(batch, N, M) is None  # y is the state sequence
    assert _ops(batch, N, M, C=torch.ones(4, M)) is None  # h @ C.T
    assert _ops(batch, N, M, C=torch.ones(N, 4, M)) is None  # (N, _, M)
    assert _ops(batch, N, M, D=torch.ones(7), out_idx=0) is None  # x.unsqueeze(-1) * D


def test_ambiguous_shapes_follow_the_reference_order():
    n = 4  # batch == N
    M = 2
    # (N, M) is matched before (batch, M): per step, not per row
    assert _ops(n, n, M, B=torch.ones(n, M), out_idx=0)[0].shape == (1, n, M)
    assert _ops(n, n, M, C=torch.ones(n, M))[1].shape == (1, n, M)
    # a 3D C whose first axis is N is (N, _, M): several outputs
    assert _ops(n, n, M, C=torch.ones(n, n, M)) is None
    # a 2D D whose first axis is N is (N, _): several outputs
    assert _ops(n, n, M, D=torch.ones(n, n), out_idx=0) is None
    x = torch.randn(n, n)
    D = torch.randn(n, n)
    assert ssm._apply_D(x, D, n, n, -1).shape == (n, n, n)
    # with batch != N the same D layout is the per-row, per-step feedthrough
    x = torch.randn(3, 5)
    D = torch.randn(3, 5)
    torch.testing.assert_close(ssm._apply_D(x, D, 3, 5, -1), D * x)
