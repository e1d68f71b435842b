"""Writes the golden fixtures under tests/golden/ (run from the repo root:
python tests/golden/make_golden.py).

The expected outputs are computed by independent brute force, not by the
oracle: the selection by walking clusters sorted with Python's sort on
(value descending, +0 above -0, index ascending); the attention by an
explicit per-query softmax over the listed key rows in fp64.  The reference
operator itself cannot run here (CUDA sm_90a only), so these fixtures pin
both the oracle and the HIP kernels to the stated semantics.
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
C = 2048


def brute_select(row, sizes, ns):
    items = []
    for c in range(C):
        v = float(row[c])
        neg0 = 1 if (v == 0.0 and math.copysign(1.0, v) < 0) else 0
        items.append((-v, neg0, c))
    items.sort()
    sel = np.zeros(C, dtype=bool)
    cum = 0
    for _, _, c in items:
        sel[c] = True
        cum += int(sizes[c])
        if cum >= ns:
            break
    return sel, cum


def pack(sel):
    """bool [..., 2048] -> LSB-first int32 words, cluster c = bit c & 31 of word c >> 5."""
    flat = sel.reshape(-1, C)
    out = np.zeros((flat.shape[0], C // 32), dtype=np.uint32)
    for i in range(flat.shape[0]):
        for c in np.nonzero(flat[i])[0]:
            out[i, c >> 5] |= np.uint32(1) << np.uint32(c & 31)
    return out.reshape(sel.shape[:-1] + (C // 32,)).view(np.int32)


def select_cases():
    rng = np.random.default_rng(2024)
    N, CQ = 128, 6
    cases = {}
    for kind in ("normal", "coarse", "signedzero", "zeros"):
        sizes = rng.multinomial(N, np.ones(C) / C).astype(np.int32)
        if kind == "zeros":
            sizes[:] = 0
            sizes[rng.choice(C, 20, replace=False)] = 1
            sizes[7] += N - sizes.sum()
        if kind == "normal":
            gl = rng.normal(0, 1, (1, N, C)).astype(np.float16)
        elif kind == "coarse":
            gl = (np.round(rng.normal(0, 1, (1, N, C)) * 4) / 4).astype(np.float16)
        elif kind == "signedzero":
            gl = rng.choice(np.array([0.0, -0.0, 1.0, -1.0], dtype=np.float16), (1, N, C))
        else:
            gl = rng.normal(0, 1, (1, N, C)).astype(np.float16)
        qlab = rng.integers(0, CQ - 1, N)
        qperm = np.argsort(qlab, kind="stable").astype(np.int32)
        qcounts = np.bincount(qlab, minlength=CQ).astype(np.int32)
        cases[kind + "_gl"] = gl
        cases[kind + "_kcounts"] = sizes[None]
        cases[kind + "_qperm"] = qperm[None]
        cases[kind + "_qcounts"] = qcounts[None]
        for ns in (1, 17, N):
            sel = np.zeros((N, C), dtype=bool)
            rowcnt = np.zeros(N, dtype=np.int32)
            for i in range(N):
                sel[i], rowcnt[i] = brute_select(gl[0, i], sizes, ns)
            uni = np.zeros((CQ, C), dtype=bool)
            for t in range(CQ):
                uni[t] = sel[qlab == t].any(0) if (qlab == t).any() else False
            key = f"{kind}_ns{ns}"
            cases[key + "_unip"] = pack(uni)[None]
            cases[key + "_rowcnt"] = rowcnt[None]
    np.savez_compressed(os.path.join(HERE, "select_golden.npz"), **cases)


def attention_case():
    rng = np.random.default_rng(7)
    H, N, CQ = 1, 256, 4
    q = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    k = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    v = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    klab = rng.integers(0, 40, N)
    kperm = np.argsort(klab, kind="stable").astype(np.int32)
    kcounts = np.bincount(klab, minlength=C).astype(np.int32)
    qlab = rng.integers(0, CQ, N)
    qperm = np.argsort(qlab, kind="stable").astype(np.int32)
    qcounts = np.bincount(qlab, minlength=CQ).astype(np.int32)
    uni = np.zeros((CQ, C), dtype=bool)
    uni[0, [1, 5, 9, 33]] = True
    uni[1, :40] = True            # every non-empty cluster: dense attention
    uni[3, [2]] = True            # cluster 2 is the only one
    # uni[2] empty -> zeros, lse = -inf
    kstart = np.concatenate([[0], np.cumsum(kcounts)])
    kp = k[0][kperm]
    vp = v[0][kperm]
    out = np.zeros((N, 128))
    lse = np.full(N, -np.inf)
    qoff = np.concatenate([[0], np.cumsum(qcounts)])
    for t in range(CQ):
        rows = [r for c in range(C) if uni[t, c] for r in range(kstart[c], kstart[c + 1])]
        for j in range(qoff[t], qoff[t + 1]):
            if not rows:
                continue
            qi = q[0, qperm[j]].astype(np.float64)
            s = np.array([qi @ kp[r].astype(np.float64) for r in rows]) / math.sqrt(128)
            e = np.exp(s - s.max())
            out[j] = (e[:, None] * vp[rows].astype(np.float64)).sum(0) / e.sum()
            lse[j] = (s.max() + math.log(e.sum())) / math.log(2)
    np.savez_compressed(os.path.join(HERE, "attention_golden.npz"), q=q, kp=kp[None], vp=vp[None],
                        kcounts=kcounts[None], qperm=qperm[None], qcounts=qcounts[None],
                        unip=pack(uni)[None], out=out[None], lse=lse[None])


if __name__ == "__main__":
    select_cases()
    attention_case()
