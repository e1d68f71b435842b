"""The oracle's structure-rebuilding call spread over host processes.

TEST INFRASTRUCTURE ONLY (the CPU baseline of ``bench.py``): the same
functions of ``t2t_oracle`` as ``full_call``, with the row-parallel stages
split over a fork-based process pool:

* scores + per-row selection over chunks of rows (select_rows, the largest
  stage), the union ORed in the parent from the packed row selections;
* exact attention over chunks of query clusters;
* residual + merge over chunks of sorted rows.

The k-means maintenance runs in the parent (its per-cluster sums are
sequential by definition).  The result equals ``full_call`` to fp64 rounding
(tests/test_oracle_parallel.py).
"""
from __future__ import annotations

import multiprocessing as mp

import numpy as np

from . import t2t_oracle as O

_G: dict = {}     # inputs shared with the forked workers (copy on write)


def _select_chunk(args):
    h, lo, hi, ns = args
    g = _G
    gl = O.scores(g["QU"][h][lo:hi][None], g["cks"][h][None])[0]
    sel, rc = O.select_rows(gl, g["kcounts"][h], ns)
    return h, lo, np.packbits(sel, axis=1, bitorder="little"), rc


def _attn_chunk(args):
    h, clusters = args
    g = _G
    out, lse = O.tile_attention(g["q"], g["kp"], g["V_sorted"], g["qcounts"], g["kcounts"],
                                g["unip"], g["qperm"], heads=[h], clusters=clusters)
    qoff = O.exclusive_scan(g["qcounts"][h])
    lo = int(qoff[clusters[0]])
    hi = int(qoff[clusters[-1]] + g["qcounts"][h, clusters[-1]])
    return h, lo, out[h, lo:hi], lse[h, lo:hi]


def _merge_chunk(args):
    h, lo, hi, tailw = args
    g = _G
    out = O.tail_merge(g["attn_out"], g["attn_lse"], g["QU"], g["cks"], g["sumv"], g["kcounts"],
                       g["unip"], g["qlab"], g["qperm"], g["lam"], tailw, heads=[h],
                       rows=slice(lo, hi))
    orig = g["qperm"][h][lo:hi]
    return h, orig, out[h, orig]


def _run(workers, fn, jobs):
    ctx = mp.get_context("fork")
    with ctx.Pool(workers) as pool:
        return pool.map(fn, jobs, chunksize=1)


def full_call_pool(q, k, v, state, ns, CQ, *, workers, pin_tail=0, tailw=1.0, chunks=4):
    """``t2t_oracle.full_call`` on ``workers`` processes; returns the output
    (fp64 [H, N, 128], original order)."""
    H, N, _ = q.shape
    QU = O.project(q, state["Uq"])
    KU = O.project(k, state["Uk"])
    km = O.kmeans_maintain(QU, KU, v, state["cq"], state["ck"], pin_tail=pin_tail)
    _, cks = O.scale_centroids(km["ck2"])
    _G.clear()
    _G.update(q=q, QU=QU, cks=cks, **km)
    n_jobs = max(1, workers * chunks // H)
    bounds = np.linspace(0, N, n_jobs + 1).astype(int)
    sel = np.zeros((H, N, O.C_KEYS // 8), dtype=np.uint8)
    rowcnt = np.zeros((H, N), dtype=np.int32)
    for h, lo, bits, rc in _run(workers, _select_chunk,
                                [(h, bounds[i], bounds[i + 1], ns) for h in range(H)
                                 for i in range(n_jobs)]):
        sel[h, lo:lo + len(rc)] = bits
        rowcnt[h, lo:lo + len(rc)] = rc
    unip = np.zeros((H, CQ, O.C_KEYS // 32), dtype=np.int32)
    for h in range(H):
        off = O.exclusive_scan(km["qcounts"][h])
        for t in range(CQ):
            rows = km["qperm"][h, off[t]: off[t] + km["qcounts"][h, t]]
            if rows.size:
                unip[h, t] = np.bitwise_or.reduce(sel[h, rows], axis=0).view(np.int32)
    if pin_tail:
        unip = O.or_pin_tail(unip)
    kp = np.stack([k[h][km["kperm"][h]] for h in range(H)])
    _G.update(kp=kp, unip=unip)
    live = [(h, [t for t in range(CQ) if km["qcounts"][h, t] > 0]) for h in range(H)]
    attn_jobs = []
    for h, ts in live:
        for part in np.array_split(np.array(ts), n_jobs):
            if part.size:
                attn_jobs.append((h, part.tolist()))
    ao = np.zeros((H, N, 128), dtype=np.float64)
    lse = np.full((H, N), -np.inf, dtype=np.float64)
    for h, lo, o, l in _run(workers, _attn_chunk, attn_jobs):
        ao[h, lo:lo + len(l)] = o
        lse[h, lo:lo + len(l)] = l
    _G.update(attn_out=ao, attn_lse=lse)
    out = np.zeros((H, N, 128), dtype=np.float64)
    for h, orig, o in _run(workers, _merge_chunk,
                           [(h, bounds[i], bounds[i + 1], tailw) for h in range(H)
                            for i in range(n_jobs)]):
        out[h, orig] = o
    _G.clear()
    return out
