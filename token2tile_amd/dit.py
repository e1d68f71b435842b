"""Wan2.1-architecture DiT forward with the Token2Tile attention backend.

End-to-end harness for the operator: a diffusion transformer with the Wan2.1
block structure (adaLN modulation, q/k RMSNorm, 3-D rotary embedding,
cross-attention to a text context, GELU feed-forward) and random bf16 weights.
Its self-attention runs either dense (torch SDPA) or through
``token2tile_amd.backend.t2t_attn.T2TAttentionImpl`` with the backend's budget
profile, dense prefix and mask-refresh reuse, so one denoising step can be
timed both ways on the same weights and inputs.

``python -m token2tile_amd.dit`` prints one JSON line with the per-step times
at the Wan2.1-14B 720p shape (40 blocks, hidden 5120, 40 heads, FFN 13824,
75,600 latent tokens, 512 context tokens).
"""
from __future__ import annotations

import argparse
import json
import math
import sys
import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class DiTConfig:
    """Block structure of Wan2.1-T2V-14B."""

    blocks: int = 40
    hidden: int = 5120
    heads: int = 40
    ffn: int = 13824
    context_tokens: int = 512
    grid: tuple[int, int, int] = (21, 45, 80)  # latent frames x height x width (720p)
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def tokens(self) -> int:
        f, h, w = self.grid
        return f * h * w


def rope_tables(cfg: DiTConfig, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin [N, head_dim / 2] of the 3-D rotary embedding: the rotary
    pairs of a head are split between the frame, height and width positions
    (d - 4 (d // 6), 2 (d // 6), 2 (d // 6) channels, as in Wan2.1)."""
    d = cfg.head_dim
    parts = [d - 4 * (d // 6), 2 * (d // 6), 2 * (d // 6)]
    f, h, w = cfg.grid
    pos = torch.stack(torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w),
                                     indexing="ij"), dim=-1).reshape(-1, 3).to(device)
    angles = []
    for axis, ch in enumerate(parts):
        inv = 1.0 / (10000.0 ** (torch.arange(0, ch, 2, device=device, dtype=torch.float64) / ch))
        angles.append(pos[:, axis:axis + 1].double() * inv[None])
    ang = torch.cat(angles, dim=1)                  # [N, d / 2]
    return ang.cos().float(), ang.sin().float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, N, H, d]: rotate channel pairs (2i, 2i + 1) by the position angles."""
    xf = x.float().unflatten(-1, (-1, 2))
    x0, x1 = xf[..., 0], xf[..., 1]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    out = torch.stack((x0 * c - x1 * s, x0 * s + x1 * c), dim=-1).flatten(-2)
    return out.to(x.dtype)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * weight


class Block(torch.nn.Module):
    def __init__(self, cfg: DiTConfig, index: int, attn_impl=None):
        super().__init__()
        D, Fh = cfg.hidden, cfg.ffn
        self.cfg = cfg
        self.index = index
        self.modulation = torch.nn.Parameter(torch.randn(1, 6, D) / D ** 0.5)
        self.q = torch.nn.Linear(D, D)
        self.k = torch.nn.Linear(D, D)
        self.v = torch.nn.Linear(D, D)
        self.o = torch.nn.Linear(D, D)
        self.norm_q = torch.nn.Parameter(torch.ones(D))
        self.norm_k = torch.nn.Parameter(torch.ones(D))
        self.norm3 = torch.nn.LayerNorm(D, eps=cfg.eps)
        self.cq = torch.nn.Linear(D, D)
        self.ck = torch.nn.Linear(D, D)
        self.cv = torch.nn.Linear(D, D)
        self.co = torch.nn.Linear(D, D)
        self.cnorm_q = torch.nn.Parameter(torch.ones(D))
        self.cnorm_k = torch.nn.Parameter(torch.ones(D))
        self.ffn1 = torch.nn.Linear(D, Fh)
        self.ffn2 = torch.nn.Linear(Fh, D)
        self.attn_impl = attn_impl  # None: dense SDPA

    def self_attention(self, x, rope, attn_metadata):
        B, N, D = x.shape
        H, d = self.cfg.heads, self.cfg.head_dim
        q = rms_norm(self.q(x), self.norm_q, self.cfg.eps).view(B, N, H, d)
        k = rms_norm(self.k(x), self.norm_k, self.cfg.eps).view(B, N, H, d)
        v = self.v(x).view(B, N, H, d)
        q, k = apply_rope(q, *rope), apply_rope(k, *rope)
        if self.attn_impl is None:
            o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                               v.transpose(1, 2)).transpose(1, 2)
        else:
            o = self.attn_impl.forward(q, k, v, attn_metadata)
        return self.o(o.reshape(B, N, D))

    def cross_attention(self, x, ctx):
        B, N, D = x.shape
        H, d = self.cfg.heads, self.cfg.head_dim
        q = rms_norm(self.cq(x), self.cnorm_q, self.cfg.eps).view(B, N, H, d).transpose(1, 2)
        k = rms_norm(self.ck(ctx), self.cnorm_k, self.cfg.eps).view(B, -1, H, d).transpose(1, 2)
        v = self.cv(ctx).view(B, -1, H, d).transpose(1, 2)
        o = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(B, N, D)
        return self.co(o)

    def forward(self, x, t_emb, ctx, rope, attn_metadata):
        e = (self.modulation + t_emb[:, None, :]).chunk(6, dim=1)  # 6 x [B, 1, D]
        D = self.cfg.hidden
        h = F.layer_norm(x, (D,), eps=self.cfg.eps) * (1 + e[1]) + e[0]
        x = x + self.self_attention(h, rope, attn_metadata) * e[2]
        x = x + self.cross_attention(self.norm3(x), ctx)
        h = F.layer_norm(x, (D,), eps=self.cfg.eps) * (1 + e[4]) + e[3]
        x = x + self.ffn2(F.gelu(self.ffn1(h), approximate="tanh")) * e[5]
        return x


class WanDiT(torch.nn.Module):
    """The block stack (patch embedding, time embedding MLP and the output
    head are outside the attention path and omitted; the latent enters as
    [1, N, hidden] tokens)."""

    def __init__(self, cfg: DiTConfig, sparse: bool, device, dtype=torch.bfloat16, tie=0.0):
        super().__init__()
        self.cfg = cfg
        impls = [None] * cfg.blocks
        if sparse:
            from token2tile_amd.backend.t2t_attn import T2TAttentionImpl
            impls = [T2TAttentionImpl(cfg.heads, cfg.head_dim, False, 1.0 / math.sqrt(cfg.head_dim),
                                      prefix=f"blocks.{i}.self_attn.attn") for i in range(cfg.blocks)]
        with torch.device(device):
            self.blocks = torch.nn.ModuleList(Block(cfg, i, impls[i]) for i in range(cfg.blocks))
        for m in self.modules():
            if isinstance(m, torch.nn.Linear):
                torch.nn.init.normal_(m.weight, std=m.in_features ** -0.5)
                torch.nn.init.zeros_(m.bias)
        if tie > 0:
            # self-attention key weights tied to the query weights (same scale):
            # W_k = tie W_q + sqrt(1 - tie^2) W_k, so q_i . k_j is large for
            # similar tokens and attention follows the latent's structure
            with torch.no_grad():
                for blk in self.blocks:
                    blk.k.weight.mul_(math.sqrt(1.0 - tie * tie)).add_(tie * blk.q.weight)
        self.to(dtype)
        self.rope = rope_tables(cfg, device)

    @torch.no_grad()
    def forward(self, x, t_emb, ctx, metadata_for_layer=None):
        for blk in self.blocks:
            md = metadata_for_layer(blk.index) if metadata_for_layer is not None else None
            x = blk(x, t_emb, ctx, self.rope, md)
        return x


def smooth_latent(cfg: DiTConfig, g, device, components=32, noise=0.3):
    """[1, N, hidden] tokens that vary smoothly over the (frame, height,
    width) grid: a sum of low-frequency plane waves, each along its own
    random direction of the hidden space, plus white noise."""
    f, h, w = cfg.grid
    pos = torch.stack(torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w),
                                     indexing="ij"), dim=-1).reshape(-1, 3).to(device).float()
    pos = pos / torch.tensor([f, h, w], device=device, dtype=torch.float32)
    freq = 3.0 * torch.randn(3, components, generator=g, device=device)
    phase = 2 * math.pi * torch.rand(components, generator=g, device=device)
    dirs = torch.randn(components, cfg.hidden, generator=g, device=device)
    waves = torch.sin(2 * math.pi * pos @ freq + phase)                 # [N, components]
    x = waves @ dirs / math.sqrt(components)
    x += noise * torch.randn(x.shape, generator=g, device=device)
    return x[None].to(torch.bfloat16)


def run(cfg: DiTConfig, steps, device, *, sparse: bool, profile="auto", budget_kw=None, seed=0,
        structured=False):
    """Time one forward (one CFG branch) of the block stack per denoising step
    index in ``steps``; returns {step: ms}.  With ``sparse`` the self-attention
    goes through the T2T backend, whose dense prefix, budget windows and
    mask-refresh schedule follow the step index.  ``structured``: key weights
    tied to the query weights (0.9) and a spatially smooth latent, so that
    attention is local, as in trained video models (random weights and white
    noise give near-uniform attention, whose unions hold most keys)."""
    torch.manual_seed(seed)
    model = WanDiT(cfg, sparse, device, tie=0.9 if structured else 0.0)
    g = torch.Generator(device=device).manual_seed(seed + 1)
    if structured:
        x = smooth_latent(cfg, g, device)
    else:
        x = torch.randn(1, cfg.tokens, cfg.hidden, generator=g, device=device, dtype=torch.bfloat16)
    ctx = torch.randn(1, cfg.context_tokens, cfg.hidden, generator=g, device=device,
                      dtype=torch.bfloat16)
    t_emb = 0.1 * torch.randn(1, cfg.hidden, generator=g, device=device, dtype=torch.bfloat16)
    builder = cache = None
    if sparse:
        from token2tile_amd.backend.t2t_attn import T2TAttentionMetadataBuilder, T2TRequestCache
        builder, cache = T2TAttentionMetadataBuilder(), T2TRequestCache()
    times = {}
    for step in steps:
        md = None
        if sparse:
            md = builder.build(step_index=step, total_steps=50, cache=cache, profile_name=profile,
                               **(budget_kw or {}))
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        y = model(x, t_emb, ctx, (lambda i, m=md: m) if sparse else None)
        torch.cuda.synchronize(device)
        times[step] = (time.perf_counter() - t0) * 1e3
        print(f"[dit] {'t2t' if sparse else 'dense'} step {step}: {times[step]:.1f} ms",
              file=sys.stderr, flush=True)
        assert bool(torch.isfinite(y).all()), "non-finite DiT output"
    return times


WINDOWS = ((12, 21), (21, 31), (31, 41), (41, 50))  # the backend's budget windows


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--blocks", type=int, default=40)
    p.add_argument("--per-window", type=int, default=4,
                   help="sparse steps timed per budget window (after the initial step 12)")
    p.add_argument("--structured", action="store_true",
                   help="tied q/k weights and a smooth latent (local attention); default: random")
    args = p.parse_args(argv)
    if not torch.cuda.is_available():
        sys.exit("the DiT harness needs a ROCm GPU")
    dev = torch.device("cuda", 0)
    cfg = DiTConfig(blocks=args.blocks)
    dense = run(cfg, [0, 1, 2], dev, sparse=False, structured=args.structured)
    d_ms = (dense[1] + dense[2]) / 2
    torch.cuda.empty_cache()
    # step 12 fits the projections and centroids (init_state) and rebuilds;
    # then a run of consecutive steps per window, so the mask-refresh
    # schedule (one structure rebuild per 4 steps) is what gets timed
    steps = [12]
    for lo, hi in WINDOWS:
        first = lo + 1 if lo == 12 else lo
        steps += list(range(first, min(hi, first + args.per_window)))
    sparse = run(cfg, steps, dev, sparse=True, structured=args.structured)
    win_ms = []
    for lo, hi in WINDOWS:
        ts = [sparse[s] for s in steps if lo <= s < hi and s != 12]
        win_ms.append(sum(ts) / len(ts))
    n_steps = [hi - lo for lo, hi in WINDOWS]
    # step 12 (the fit + first rebuild) at its measured time, the other
    # sparse steps at their window's mean
    n_steps[0] -= 1
    t2t_total = 12 * d_ms + sparse[12] + sum(n * w for n, w in zip(n_steps, win_ms))
    out = {"metric": "Wan2.1-14B DiT denoising step (one CFG branch), ms",
           "config": {"blocks": cfg.blocks, "hidden": cfg.hidden, "heads": cfg.heads,
                      "ffn": cfg.ffn, "tokens": cfg.tokens, "context_tokens": cfg.context_tokens,
                      "dtype": "bf16",
                      "weights": "random, k tied to q (0.9), smooth latent" if args.structured
                      else "random", "attention_profile": "auto"},
           "dense_ms_per_step": round(d_ms, 1),
           "t2t_step_ms": {str(k): round(v, 1) for k, v in sparse.items()},
           "t2t_ms_per_step_by_window": [round(w, 1) for w in win_ms],
           "init_step_ms": round(sparse[12], 1),
           "schedule_50_steps_s": {"dense": round(50 * d_ms / 1e3, 2),
                                   "t2t": round(t2t_total / 1e3, 2)},
           "schedule_speedup_50_steps": round(50 * d_ms / t2t_total, 3)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
