"""Host-side pieces of the closed-loop attention adapter (CPU)."""

from __future__ import annotations

import pytest
import torch

from jointkv_amd.closed_loop_attention import AttentionWeights, relative_trajectory_attention_mse


def test_trajectory_mse_hand_worked():
    # mean((c - r)^2) = (1 + 0 + 4 + 1) / 4 = 1.5; mean(r^2) = (1 + 4 + 0 + 9) / 4 = 3.5
    r = torch.tensor([[[1.0, 2.0], [0.0, 3.0]]])
    c = torch.tensor([[[2.0, 2.0], [2.0, 2.0]]])
    assert float(relative_trajectory_attention_mse(c, r)) == pytest.approx(1.5 / 3.5)
    # a zero reference is floored at epsilon
    z = torch.zeros(1, 2, 2)
    assert float(relative_trajectory_attention_mse(c, z, epsilon=0.5)) == pytest.approx(4.0 / 0.5)
    with pytest.raises(ValueError, match="geometry"):
        relative_trajectory_attention_mse(c[0], r[0])
    with pytest.raises(ValueError, match="epsilon"):
        relative_trajectory_attention_mse(c, r, epsilon=0.0)
    # the reference side is stopped
    cg = c.clone().requires_grad_(True)
    rg = r.clone().requires_grad_(True)
    relative_trajectory_attention_mse(cg, rg).backward()
    assert rg.grad is None and cg.grad is not None


def test_attention_weights_geometry():
    w = AttentionWeights(torch.zeros(4096, 4096), torch.zeros(1024, 4096), torch.zeros(1024, 4096),
                         torch.zeros(4096, 4096))
    assert (w.query_heads, w.kv_heads) == (32, 8)
