"""Pins the oracle's exact tile attention (S5) and residual merge (S6):
an all-ones union is dense attention (torch SDPA on CPU), a one-cluster
union is a hand-sliced softmax, and the merge has closed forms at its
special cases (empty union, full union, tailw = 0)."""
import math

import numpy as np
import torch

from oracle import t2t_oracle as O


def small_structure(rng, H=1, N=512, CQ=8, CK=2048):
    klab = rng.integers(0, 64, (H, N)).astype(np.int32)     # only 64 non-empty key clusters
    kperm, kcounts = O.stable_perm(klab, CK)
    qlab = rng.integers(0, CQ, (H, N)).astype(np.int32)
    qperm, qcounts = O.stable_perm(qlab, CQ)
    return klab, kperm, kcounts, qlab, qperm, qcounts


def test_full_union_is_dense_attention():
    rng = np.random.default_rng(0)
    H, N, CQ = 1, 512, 8
    q = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    k = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    v = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    klab, kperm, kcounts, qlab, qperm, qcounts = small_structure(rng, H, N, CQ)
    unip = O.pack_bits(np.ones((H, CQ, 2048), dtype=bool))
    kp = k[0][kperm[0]][None]
    vp = v[0][kperm[0]][None]
    out, lse = O.tile_attention(q, kp, vp, qcounts, kcounts, unip, qperm)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.tensor(q, dtype=torch.float64), torch.tensor(k, dtype=torch.float64),
        torch.tensor(v, dtype=torch.float64)).numpy()
    assert np.allclose(out[0], ref[0][qperm[0]], atol=1e-10)
    s = q[0].astype(np.float64) @ k[0].astype(np.float64).T / math.sqrt(128)
    want_lse = np.log(np.exp(s).sum(1)) / math.log(2)
    assert np.allclose(lse[0], want_lse[qperm[0]], atol=1e-10)


def test_single_cluster_union_and_empty_union():
    rng = np.random.default_rng(1)
    H, N, CQ = 1, 512, 8
    q = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    k = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    v = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    klab, kperm, kcounts, qlab, qperm, qcounts = small_structure(rng, H, N, CQ)
    sel = np.zeros((H, CQ, 2048), dtype=bool)
    sel[0, 0, 5] = True          # cluster 0 attends to key cluster 5 only; others empty
    unip = O.pack_bits(sel)
    kp = k[0][kperm[0]][None]
    vp = v[0][kperm[0]][None]
    out, lse = O.tile_attention(q, kp, vp, qcounts, kcounts, unip, qperm)
    keys = np.nonzero(klab[0] == 5)[0]
    qoff = np.concatenate([[0], np.cumsum(qcounts[0])])
    for j in range(qoff[0], qoff[1]):
        i = qperm[0, j]
        s = q[0, i].astype(np.float64) @ k[0, keys].astype(np.float64).T / math.sqrt(128)
        p = np.exp(s - s.max())
        assert np.allclose(out[0, j], p @ v[0, keys].astype(np.float64) / p.sum(), atol=1e-12)
    assert np.all(out[0, qoff[1]:] == 0) and np.all(np.isneginf(lse[0, qoff[1]:]))


def _tail_inputs(rng, H=1, N=256, CQ=4):
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    cks = (rng.normal(0, 1, (H, 2048, 32)) * 0.2).astype(np.float16)
    sumv = rng.normal(0, 1, (H, 2048, 128)).astype(np.float16)
    kcounts = rng.integers(0, 4, (H, 2048)).astype(np.int32)
    qlab = rng.integers(0, CQ, (H, N)).astype(np.int32)
    qperm, qcounts = O.stable_perm(qlab, CQ)
    ao = rng.normal(0, 1, (H, N, 128))
    lse = rng.normal(3, 1, (H, N))
    lam = np.array([1.5], dtype=np.float32)
    return QU, cks, sumv, kcounts, qlab, qperm, qcounts, ao, lse, lam


def test_tail_closed_forms():
    rng = np.random.default_rng(2)
    QU, cks, sumv, kcounts, qlab, qperm, qcounts, ao, lse, lam = _tail_inputs(rng)
    CQ = qcounts.shape[1]
    # full union: exact output unchanged (written at the original row)
    full = O.pack_bits(np.ones((1, CQ, 2048), dtype=bool))
    out = O.tail_merge(ao, lse, QU, cks, sumv, kcounts, full, qlab, qperm, lam)
    assert np.array_equal(out[0][qperm[0]], ao[0])
    # tailw = 0: exact output
    half = np.zeros((1, CQ, 2048), dtype=bool)
    half[..., :1024] = True
    hp = O.pack_bits(half)
    out0 = O.tail_merge(ao, lse, QU, cks, sumv, kcounts, hp, qlab, qperm, lam, tailw=0.0)
    assert np.allclose(out0[0][qperm[0]], ao[0], atol=1e-12)
    # empty union + lse = -inf: residual only, lam * O / phi
    empty = O.pack_bits(np.zeros((1, CQ, 2048), dtype=bool))
    ninf = np.full_like(lse, -np.inf)
    oute = O.tail_merge(np.zeros_like(ao), ninf, QU, cks, sumv, kcounts, empty, qlab, qperm, lam)
    s = O.scores(QU, cks)[0].astype(np.float64)
    for i in (0, 17, 100):
        p = np.exp(s[i] - (s[i].max() + 2.0))   # the oracle shift: fp16(p) depends on it
        phi = (p * kcounts[0]).sum()
        Ov = p.astype(np.float32).astype(np.float16).astype(np.float64) @ sumv[0].astype(np.float64)
        assert np.allclose(oute[0, i], lam[0] * Ov / phi, rtol=1e-6, atol=1e-9)
    # general case: one softmax over exact part (weight e^le) and residual part
    outg = O.tail_merge(ao, lse, QU, cks, sumv, kcounts, hp, qlab, qperm, lam)
    for j in (0, 50):
        i = qperm[0, j]
        mask = half[0, qlab[0, i]]
        p = np.where(mask, 0.0, np.exp(s[i]))
        phi = (p * kcounts[0]).sum()
        Ov = (np.where(mask, 0.0, p)).astype(np.float64)
        # residual weights use fp16 p relative to a shift; compare against the shift-free form
        ex = np.exp(lse[0, j] * math.log(2))
        want = (ex * ao[0, j] + lam[0] * (Ov @ sumv[0].astype(np.float64))) / (ex + phi)
        assert np.allclose(outg[0, i], want, rtol=2e-3, atol=2e-3)
