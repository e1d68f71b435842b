"""Seeded synthetic attention inputs for the benchmark configurations.

Q and K are a 128-d Gaussian mixture (256 components with N(0, 1) means,
within-component sigma 0.3) scaled by 1/sqrt(128); V ~ N(0, 1).  The GPU
configurations add a smooth 3-D positional drift over the latent grid
(frames x height x width), which correlates neighbouring tokens.
``generate`` is deterministic for a given (seed, shape, device type): numpy
on the host for small shapes, torch's generator on the device for large
ones.
"""
from __future__ import annotations

import math

import numpy as np
import torch

CONFIGS = {
    # name: (H, N, latent grid, budget fraction, CQ)
    "cpu_plumbing": (2, 16384, (4, 64, 64), 0.05, 256),
    "wan480p": (40, 32760, (21, 30, 52), 0.05, 256),
    "wan720p": (40, 75600, (21, 45, 80), 0.015, 512),
    "h3": (48, 98304, (24, 64, 64), 0.0125, 768),
    "h3_5pct": (48, 98304, (24, 64, 64), 0.05, 768),
}


def budget(N, frac):
    return max(1, int(frac * N))


def _grid_coords(grid, N):
    f, h, w = grid
    assert f * h * w == N, (grid, N)
    t = np.arange(N)
    return np.stack([t // (h * w), (t // w) % h, t % w], 1).astype(np.float64) / np.array(
        [max(f, 1), max(h, 1), max(w, 1)], dtype=np.float64)


def generate_np(H, N, *, grid=None, seed=0, D=128, comps=256, sigma=0.3, drift=0.5,
                dtype=np.float16):
    """Host (numpy) generator: returns q, k, v [H, N, D] arrays."""
    rng = np.random.default_rng(seed)
    means = rng.normal(0, 1, (H, comps, D))
    out = []
    for which in range(2):
        lab = rng.integers(0, comps, (H, N))
        x = np.take_along_axis(means, lab[..., None], 1) + sigma * rng.normal(0, 1, (H, N, D))
        if grid is not None and drift > 0:
            xyz = _grid_coords(grid, N)
            freq = rng.normal(0, 2.0, (H, 3, 4))
            dirs = rng.normal(0, 1, (H, 4, D)) / math.sqrt(4)
            phase = np.einsum("nc,hck->hnk", xyz, freq) * 2 * math.pi
            x = x + drift * np.einsum("hnk,hkd->hnd", np.sin(phase), dirs)
        out.append((x / math.sqrt(D)).astype(dtype))
    v = rng.normal(0, 1, (H, N, D)).astype(dtype)
    return out[0], out[1], v


def generate(H, N, *, grid=None, seed=0, device="cuda", dtype=torch.bfloat16, D=128, comps=256,
             sigma=0.3, drift=0.5):
    """Device generator for large shapes: q, k, v [H, N, D] tensors."""
    g = torch.Generator(device=device).manual_seed(seed)
    f32 = torch.float32
    means = torch.randn(H, comps, D, generator=g, device=device, dtype=f32)
    xyz = None
    if grid is not None and drift > 0:
        xyz = torch.tensor(_grid_coords(grid, N), device=device, dtype=f32)
    outs = []
    for _ in range(2):
        lab = torch.randint(0, comps, (H, N), generator=g, device=device)
        x = torch.gather(means, 1, lab[..., None].expand(H, N, D))
        x += sigma * torch.randn(H, N, D, generator=g, device=device, dtype=f32)
        if xyz is not None:
            freq = 2.0 * torch.randn(H, 3, 4, generator=g, device=device, dtype=f32)
            dirs = torch.randn(H, 4, D, generator=g, device=device, dtype=f32) / 2.0
            phase = torch.einsum("nc,hck->hnk", xyz, freq) * (2 * math.pi)
            x += drift * torch.einsum("hnk,hkd->hnd", torch.sin(phase), dirs)
        outs.append((x / math.sqrt(D)).to(dtype))
        del x
    v = torch.randn(H, N, D, generator=g, device=device, dtype=f32).to(dtype)
    return outs[0], outs[1], v
