"""The Wan2.1-architecture DiT harness: rotary embedding and RMSNorm closed
forms, block shapes on the CPU; on the GPU, the T2T backend inside the block
stack (dense-prefix step identical to the dense model, sparse steps close to
it)."""
import math

import pytest
import torch

from token2tile_amd import dit


def test_rope_tables_and_rotation():
    cfg = dit.DiTConfig(blocks=1, hidden=256, heads=2, ffn=64, context_tokens=4, grid=(2, 3, 4))
    cos, sin = dit.rope_tables(cfg, "cpu")
    assert cos.shape == (24, 64) and sin.shape == (24, 64)
    # channel split 44 / 42 / 42 (pairs 22 / 21 / 21): frame, height, width
    d = cfg.head_dim
    assert d - 4 * (d // 6) == 44
    pos = 1 * 12 + 2 * 4 + 3  # frame 1, row 2, column 3
    ang = torch.atan2(sin[pos], cos[pos])
    inv_f = 1.0 / 10000 ** (torch.arange(0, 44, 2, dtype=torch.float64) / 44)
    assert torch.allclose(ang[:22].double(), torch.remainder(1 * inv_f + math.pi, 2 * math.pi) - math.pi,
                          atol=1e-5)
    # rotation preserves the norm of every channel pair and is the identity at position 0
    x = torch.randn(1, 24, 2, d)
    y = dit.apply_rope(x, cos, sin)
    assert torch.allclose(y[:, 0], x[:, 0])
    assert torch.allclose(x.unflatten(-1, (-1, 2)).norm(dim=-1), y.unflatten(-1, (-1, 2)).norm(dim=-1),
                          atol=1e-5)


def test_rms_norm():
    x = torch.randn(3, 7, 16)
    w = torch.rand(16) + 0.5
    y = dit.rms_norm(x, w, 1e-6)
    ref = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    assert torch.allclose(y, ref, atol=1e-5)


def test_dense_block_cpu():
    cfg = dit.DiTConfig(blocks=2, hidden=256, heads=2, ffn=128, context_tokens=8, grid=(2, 4, 4))
    torch.manual_seed(0)
    model = dit.WanDiT(cfg, sparse=False, device="cpu", dtype=torch.float32)
    x = torch.randn(1, cfg.tokens, cfg.hidden)
    y = model(x, 0.1 * torch.randn(1, cfg.hidden), torch.randn(1, 8, cfg.hidden))
    assert y.shape == x.shape and bool(torch.isfinite(y).all())


@pytest.mark.gpu
def test_sparse_block_stack(dev):
    cfg = dit.DiTConfig(blocks=2, hidden=12 * 128, heads=12, ffn=2048, context_tokens=64,
                        grid=(4, 32, 32))
    budget = dict(ns_base=600, dense_prefix_steps=1, cq=32, ck=2048,
                  step_profile=(1.0, 1.0, 1.0, 1.0), layer_profile=(1.0,) * 6,
                  cfg_mult=(1.0, 1.0))
    steps = [0, 1, 2, 3]
    t_dense = dit.run(cfg, steps, dev, sparse=False)
    t_sparse = dit.run(cfg, steps, dev, sparse=True, profile="manual", budget_kw=budget)
    assert set(t_dense) == set(t_sparse) == set(steps)

    # outputs: the dense-prefix step of the sparse model is the dense model
    torch.manual_seed(0)
    dense = dit.WanDiT(cfg, sparse=False, device=dev)
    torch.manual_seed(0)
    sparse = dit.WanDiT(cfg, sparse=True, device=dev)
    from token2tile_amd.backend.t2t_attn import T2TAttentionMetadataBuilder, T2TRequestCache
    b, cache = T2TAttentionMetadataBuilder(), T2TRequestCache()
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(1, cfg.tokens, cfg.hidden, generator=g, device=dev, dtype=torch.bfloat16)
    ctx = torch.randn(1, 64, cfg.hidden, generator=g, device=dev, dtype=torch.bfloat16)
    t = 0.1 * torch.randn(1, cfg.hidden, generator=g, device=dev, dtype=torch.bfloat16)
    yd = dense(x, t, ctx)
    for step in (0, 1, 2):
        md = b.build(step_index=step, total_steps=50, cache=cache, profile_name="manual", **budget)
        ys = sparse(x, t, ctx, lambda i, m=md: m)
        if step == 0:
            assert torch.equal(ys, yd)
        else:
            assert bool(torch.isfinite(ys).all())
            c = torch.nn.functional.cosine_similarity(ys.float().flatten(), yd.float().flatten(), dim=0)
            assert c > 0.98
