"""Host-side argument checks of the operator surface that run before any
device work (no GPU needed)."""
import pytest
import torch

from token2tile_amd import deploy_step as DS


def test_online_u_rejects_nonfinite_and_names_heads():
    q = torch.zeros(3, 10, 128)
    q[2, 3, 4] = float("nan")
    q[0, 1, 1] = float("inf")
    with pytest.raises(RuntimeError, match=r"q \(3, 10, 128\) holds 2 non-finite values, in heads \[0, 2\]"):
        DS.online_u(q, torch.zeros_like(q))
    k = torch.zeros(3, 10, 128)
    k[1, 0, 0] = float("-inf")
    with pytest.raises(RuntimeError, match=r"online_u: k .* in heads \[1\]"):
        DS.online_u(torch.zeros_like(k), k)


def test_fused_update_vstats_rejects_unsupported_widths():
    lab = torch.zeros(1, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="ku must be"):
        DS.fused_update_vstats(torch.zeros(1, 8, 16, dtype=torch.float16), lab,
                               torch.zeros(1, 4, 16, dtype=torch.float16))
    with pytest.raises(ValueError, match="v must be"):
        DS.fused_update_vstats(torch.zeros(1, 8, 32, dtype=torch.float16), lab,
                               torch.zeros(1, 4, 32, dtype=torch.float16),
                               torch.zeros(1, 8, 64, dtype=torch.float16))


def test_eigh_robust_matches_eigh_on_host():
    a = torch.randn(2, 6, 6, dtype=torch.float64)
    m = a @ a.transpose(1, 2)
    e, v = DS._eigh_robust(m)
    assert torch.allclose(v @ torch.diag_embed(e) @ v.transpose(1, 2), m, atol=1e-10)
