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


@pytest.mark.gpu
@pytest.mark.parametrize("structured", [False, True], ids=["random", "structured"])
def test_wan14b_720p_stack_dense_vs_t2t(dev, metrics, structured):
    """BASELINE config 5 at full size: the Wan2.1-14B block stack (40 blocks,
    hidden 5120, 40 heads, FFN 13824, 75,600 video + 512 text tokens, random
    bf16 weights), one dense step and two T2T steps through the backend with
    the built-in 720p profile: step 12 (projection fit + first structure
    rebuild) and step 13 (a mask_refresh=4 reuse step).  Checks a finite
    output, the T2T output against the dense one (cosine), that the fitted
    state persists from step 12 to step 13 without a refit, and records both
    step times.  ``structured``: key weights tied to the query weights and a
    spatially smooth latent, so that attention is local (smaller unions)."""
    import time
    cfg = dit.DiTConfig()
    assert (cfg.blocks, cfg.hidden, cfg.heads, cfg.ffn, cfg.tokens) == (40, 5120, 40, 13824, 75600)
    torch.manual_seed(0)
    model = dit.WanDiT(cfg, sparse=True, device=dev, tie=0.9 if structured else 0.0)
    impls = [blk.attn_impl for blk in model.blocks]
    g = torch.Generator(device=dev).manual_seed(1)
    if structured:
        x = dit.smooth_latent(cfg, g, dev)
    else:
        x = torch.randn(1, cfg.tokens, cfg.hidden, generator=g, device=dev, dtype=torch.bfloat16)
    tag = "dit720p_structured" if structured else "dit720p"
    ctx = torch.randn(1, cfg.context_tokens, cfg.hidden, generator=g, device=dev,
                      dtype=torch.bfloat16)
    t = 0.1 * torch.randn(1, cfg.hidden, generator=g, device=dev, dtype=torch.bfloat16)

    def timed(fn):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        y = fn()
        torch.cuda.synchronize(dev)
        return y, (time.perf_counter() - t0) * 1e3

    for blk in model.blocks:
        blk.attn_impl = None
    timed(lambda: model(x, t, ctx))                     # warm-up (library set-up)
    yd, dense_ms = timed(lambda: model(x, t, ctx))
    print(f"[{tag}] dense step {dense_ms:.0f} ms", flush=True)
    for blk, impl in zip(model.blocks, impls):
        blk.attn_impl = impl
    from token2tile_amd.backend.t2t_attn import T2TAttentionMetadataBuilder, T2TRequestCache
    builder, cache = T2TAttentionMetadataBuilder(), T2TRequestCache()
    outs, ms = {}, {}
    for step in (12, 13):
        md = builder.build(step_index=step, total_steps=50, cache=cache, profile_name="auto")
        outs[step], ms[step] = timed(lambda m=md: model(x, t, ctx, lambda i: m))
        print(f"[{tag}] t2t step {step} {ms[step]:.0f} ms", flush=True)
        if step == 12:
            assert len(cache.states) == cfg.blocks          # one fitted state per layer
            fitted = {k_: st["Uq"] for k_, st in cache.states.items()}
    assert all(cache.states[k_]["Uq"] is u for k_, u in fitted.items())   # no refit at step 13
    for step, y in outs.items():
        assert bool(torch.isfinite(y).all())
        cs = torch.nn.functional.cosine_similarity(y.float().flatten(), yd.float().flatten(), dim=0)
        metrics[f"{tag}_cos_t2t_step{step}_vs_dense"] = round(float(cs), 5)
        assert cs > 0.999, (step, float(cs))
    metrics[f"{tag}_dense_step_ms"] = round(dense_ms, 1)
    metrics[f"{tag}_t2t_step12_fit_rebuild_ms"] = round(ms[12], 1)
    metrics[f"{tag}_t2t_step13_reuse_ms"] = round(ms[13], 1)
    metrics[f"{tag}_step13_speedup_vs_dense"] = round(dense_ms / ms[13], 3)
