"""The committed golden fixtures (tests/golden/, written by brute force by
tests/golden/make_golden.py) against the oracle (CPU) and the HIP kernels
(GPU): selection/union bit-exact, attention within tolerance."""
import os

import numpy as np
import pytest

from oracle import t2t_oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KINDS = ("normal", "coarse", "signedzero", "zeros")
NS = (1, 17, 128)


def load(name):
    return np.load(os.path.join(HERE, name))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("ns", NS)
def test_oracle_select_matches_golden(kind, ns):
    z = load("select_golden.npz")
    unip, rowcnt = O.select_union(z[kind + "_gl"], z[kind + "_kcounts"], z[kind + "_qperm"],
                                  z[kind + "_qcounts"], ns)
    assert np.array_equal(unip, z[f"{kind}_ns{ns}_unip"])
    assert np.array_equal(rowcnt, z[f"{kind}_ns{ns}_rowcnt"])


def test_oracle_attention_matches_golden():
    z = load("attention_golden.npz")
    out, lse = O.tile_attention(z["q"], z["kp"], z["vp"], z["qcounts"], z["kcounts"], z["unip"],
                                z["qperm"])
    assert np.allclose(out, z["out"], atol=1e-10)
    fin = np.isfinite(z["lse"])
    assert np.array_equal(fin, np.isfinite(lse))
    assert np.allclose(lse[fin], z["lse"][fin], atol=1e-10)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", KINDS)
def test_hip_select_matches_golden(dev, kind):
    import torch
    from token2tile_amd import ops
    z = load("select_golden.npz")
    t = {k: torch.from_numpy(z[kind + "_" + k]).to(dev) for k in ("gl", "kcounts", "qperm", "qcounts")}
    for ns in NS:
        ns_t = torch.tensor(ns, dtype=torch.int32, device=dev)
        unip, rowcnt = ops.select_union(t["gl"], t["kcounts"], t["qperm"], t["qcounts"], ns_t)
        assert np.array_equal(unip.cpu().numpy(), z[f"{kind}_ns{ns}_unip"]), ns
        assert np.array_equal(rowcnt.cpu().numpy(), z[f"{kind}_ns{ns}_rowcnt"]), ns


@pytest.mark.gpu
def test_hip_attention_matches_golden(dev):
    import torch
    from token2tile_amd import ops
    z = load("attention_golden.npz")
    g = {k: torch.from_numpy(z[k]).to(dev) for k in ("q", "kp", "vp", "kcounts", "qperm", "qcounts",
                                                       "unip")}
    N = z["q"].shape[1]
    plan = ops.tile_plan(g["qcounts"], g["kcounts"], g["unip"], N)
    ao, lse = ops.tile_attn_exact(g["q"], g["kp"], g["vp"], g["kcounts"], g["unip"], g["qperm"],
                                  plan)
    assert np.abs(ao.float().cpu().numpy() - z["out"]).max() < 4e-3
    got = lse.cpu().numpy()
    fin = np.isfinite(z["lse"])
    assert np.array_equal(fin, np.isfinite(got))
    assert np.abs(got[fin] - z["lse"][fin]).max() < 2e-3
