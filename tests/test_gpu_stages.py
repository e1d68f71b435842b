"""Stage-by-stage parity of the HIP kernels with the CPU oracle.

Integer / index work is compared bit-exactly given identical inputs; MMA
products (projection, scores) within 1 fp16 ulp; attention outputs within
the stated tolerances.  Each stage is fed the same inputs on both sides
(the GPU's previous-stage outputs where a stage has an MMA-rounded input).
"""
import math
import zlib

import numpy as np
import pytest
import torch

from oracle import t2t_oracle as O

pytestmark = pytest.mark.gpu


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def c(t):
    return t.detach().cpu().numpy()


def within_ulp(a16, b16, ulps=1, acc_err=2e-5):
    """|a - b| <= ulps fp16 ulp of b + the fp32 accumulation error of the
    GPU dot product (which matters where the sum cancels to a tiny value)."""
    a = a16.astype(np.float32)
    b = b16.astype(np.float32)
    sp = np.spacing(np.abs(b16.astype(np.float16))).astype(np.float32)
    return np.all(np.abs(a - b) <= ulps * sp + acc_err)


def clustered(rng, H, N, r, C, spread=0.05):
    """Points near centroids: labels are unambiguous (no near ties)."""
    cent = rng.normal(0, 1, (H, C, r)).astype(np.float16)
    lab = rng.integers(0, C, (H, N))
    x = np.take_along_axis(cent.astype(np.float64), lab[..., None], 1)
    x = (x + spread * rng.normal(0, 1, (H, N, r))).astype(np.float16)
    return x, cent, lab


# ---------------------------------------------------------------------------
def test_project_f16_bf16(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(0)
    H, N = 2, 1000
    x = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    U = (rng.normal(0, 1, (H, 128, 32)) / 8).astype(np.float16)
    out = c(ops.project(g(x, dev), g(U, dev)))
    assert within_ulp(out, O.project(x, U))
    xb = g(x, dev).to(torch.bfloat16)
    outb = c(ops.project(xb, g(U, dev)))
    xr = c(xb.float()).astype(np.float16)          # bf16 -> fp16 as the backend cast
    assert within_ulp(outb, O.project(xr, U))


@pytest.mark.parametrize("N", [1, 31, 33, 4097])
def test_project_edge_rows_and_strides(dev, N):
    """Row counts around the 32-row blocks of the staged projection, and the
    token-major view that the backend passes (rows H * 128 apart)."""
    from token2tile_amd import ops
    rng = np.random.default_rng(100 + N)
    H = 3
    x = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    U = (rng.normal(0, 1, (H, 128, 32)) / 8).astype(np.float16)
    want = O.project(x, U)
    assert within_ulp(c(ops.project(g(x, dev), g(U, dev))), want)
    tm = g(np.ascontiguousarray(x.transpose(1, 0, 2)), dev)     # [N, H, 128]
    assert within_ulp(c(ops.project(tm.transpose(0, 1), g(U, dev))), want)


@pytest.mark.parametrize("C", [20, 600])
def test_kmeans_assignment_small_and_chunked_centroid_counts(dev, C):
    """Key clusters fewer than one 32-row block, and more than one 512-row
    staging chunk (not a multiple of 32): near-argmin labels, and the same
    outputs whatever the label buffers held."""
    from token2tile_amd import ops
    rng = np.random.default_rng(200 + C)
    H, N, CQ = 2, 3000, 40
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    KU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    cq0 = QU[:, rng.choice(N, CQ, replace=False)].copy()
    ck0 = KU[:, rng.choice(N, C, replace=False)].copy()
    V = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    args = [g(a, dev) for a in (QU, KU, V, cq0, ck0)]
    base = ops.kmm_run(*args)
    klab = c(base["klab"])
    d = O.assign_distances(KU, ck0)
    dmin = d.min(-1)
    mine = np.take_along_axis(d, klab[..., None].astype(np.int64), -1)[..., 0]
    assert np.all(mine - dmin <= 1e-4 * (1 + np.abs(dmin)))
    assert (klab != O.assign(KU, ck0)).mean() < 1e-3
    out = {"klab": g(((klab + 3) % C).astype(np.int32), dev),
           "qlab": g(rng.integers(-5, CQ + 5, (H, N)).astype(np.int32), dev)}
    again = ops.kmm_run(*args, out=out)
    for k_, v_ in base.items():
        if v_ is not None:
            assert torch.equal(v_, again[k_]), k_


def test_score_and_finalize(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(1)
    H, N = 2, 777
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    ck2 = rng.normal(0, 1, (H, 2048, 32)).astype(np.float32)
    ck16, cks = ops.centroid_finalize(g(ck2, dev))
    e16, ecks = O.scale_centroids(ck2)
    assert np.array_equal(c(ck16), e16) and np.array_equal(c(cks), ecks)
    gl = c(ops.score(g(QU, dev), cks))
    assert within_ulp(gl, O.scores(QU, ecks))


def test_gather_and_union_bit(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (3, 500, 128)).astype(np.float16)
    perm = np.stack([rng.permutation(500) for _ in range(3)]).astype(np.int32)
    out = c(ops.fast_gather(g(x, dev), g(perm, dev)))
    assert np.array_equal(out, np.stack([x[h][perm[h]] for h in range(3)]))
    xb = g(x, dev).to(torch.bfloat16)
    assert torch.equal(ops.fast_gather(xb, g(perm, dev)).cpu(),
                       torch.stack([xb[h][g(perm, dev)[h].long()] for h in range(3)]).cpu())
    u = torch.zeros(2, 5, 64, dtype=torch.int32, device=dev)
    ops.union_or_last(u)
    assert np.array_equal(c(u), O.or_pin_tail(np.zeros((2, 5, 64), dtype=np.int32)))


# ---------------------------------------------------------------------------
SEL_CASES = ["normal", "coarse", "tied", "signedzero", "zeros", "nan"]


def sel_inputs(rng, kind, H, N, CQ):
    sizes = np.stack([rng.multinomial(N, np.ones(2048) / 2048) for _ in range(H)]).astype(np.int32)
    if kind == "zeros":
        for h in range(H):
            z = rng.choice(2048, 1500, replace=False)
            moved = sizes[h, z].sum()
            sizes[h, z] = 0
            sizes[h, rng.choice(np.setdiff1d(np.arange(2048), z))] += moved
    if kind in ("normal", "zeros", "nan"):
        gl = rng.normal(0, 1, (H, N, 2048)).astype(np.float16)
        if kind == "nan":
            gl[0, :5, 100] = np.nan
    elif kind == "coarse":
        gl = (np.round(rng.normal(0, 1, (H, N, 2048)) * 4) / 4).astype(np.float16)
    elif kind == "tied":
        gl = np.full((H, N, 2048), 0.25, dtype=np.float16)
    else:
        gl = rng.choice(np.array([0.0, -0.0, 1.0, -1.0], dtype=np.float16), (H, N, 2048))
    qlab = rng.integers(0, CQ - 1, (H, N)).astype(np.int32)   # cluster CQ-1 stays empty
    qlab[:, :3] = 0
    qperm, qcounts = O.stable_perm(qlab, CQ)
    return gl, sizes, qperm, qcounts


@pytest.mark.parametrize("kind", SEL_CASES)
@pytest.mark.parametrize("ns", [1, 300, 4096])
def test_select_union_bit_exact(dev, kind, ns):
    from token2tile_amd import ops
    rng = np.random.default_rng(zlib.crc32(f"select-{kind}-{ns}".encode()))
    H, N, CQ = 2, 4096, 24
    gl, sizes, qperm, qcounts = sel_inputs(rng, kind, H, N, CQ)
    ns_t = torch.tensor(ns, dtype=torch.int32, device=dev)
    unip, rowcnt = ops.select_union(g(gl, dev), g(sizes, dev), g(qperm, dev), g(qcounts, dev), ns_t)
    eu, er = O.select_union(gl, sizes, qperm, qcounts, ns)
    assert np.array_equal(c(rowcnt), er)
    assert np.array_equal(c(unip), eu)
    u2, r2 = ops.select_union(g(gl, dev), g(sizes, dev), g(qperm, dev), g(qcounts, dev), ns_t,
                              split_cap=37)
    assert torch.equal(u2, unip) and torch.equal(r2, rowcnt)
    ub, rb = ops.select_union_bytes(g(gl, dev), g(sizes, dev), g(qperm, dev), g(qcounts, dev), ns_t)
    assert np.array_equal(c(ub).astype(bool), O.unpack_bits(eu))


# alternating_scale: consecutive rows (in the order the kernels walk them)
# differ in score scale by 2500x, so the lower bound carried over from the
# previous row is far off and the selection must fall back to a full pass
# all_tied: every centroid equal, so every score of a row ties (2048 candidates,
# more than a row's list holds, and more tied clusters than the candidate
# path takes: the full-row path).  coarse: centroids on a coarse grid, so a
# few clusters tie at the crossing key (the tie path on candidates).
# jumps: row scales that move the crossing key by a few hundred keys between
# consecutive rows (windows above and below the predicted one) and by more
# than the batch floor margin between batches (rows below the floor).
FUSED_CASES = ["normal", "tied_centroids", "zeros", "one_per_cluster", "alternating_scale",
               "all_tied", "coarse", "jumps"]


@pytest.mark.parametrize("kind", FUSED_CASES)
@pytest.mark.parametrize("ns", [1, 300, 3333])
def test_score_select_fused_matches_split(dev, kind, ns):
    """The fused scoring + selection equals t2t_score + t2t_select_run_packed
    bit for bit, and the selection matches the oracle on those scores."""
    from token2tile_amd import ops
    rng = np.random.default_rng(zlib.crc32(f"fused-{kind}-{ns}".encode()))
    H, N, CQ = 2, 3333, 24                      # N not a multiple of the 128-row block
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    ck2 = rng.normal(0, 0.5, (H, 2048, 32)).astype(np.float32)
    if kind == "tied_centroids":                 # duplicated centroids -> exactly tied scores
        ck2[:, 1024:] = ck2[:, :1024]
    if kind == "all_tied":
        ck2[:] = ck2[:, :1]
    if kind == "coarse":
        ck2 = (np.round(ck2 * 2) / 2).astype(np.float32)
        QU = (np.round(QU.astype(np.float32) * 2) / 2).astype(np.float16)
    sizes = np.stack([rng.multinomial(N, np.ones(2048) / 2048) for _ in range(H)]).astype(np.int32)
    if kind == "zeros":                         # 1500 empty key clusters, same key total
        for h in range(H):
            z = rng.choice(2048, 1500, replace=False)
            moved = sizes[h, z].sum()
            sizes[h, z] = 0
            sizes[h, rng.choice(np.setdiff1d(np.arange(2048), z))] += moved
    if kind == "one_per_cluster":
        CQ = 512
        qlab = np.stack([rng.permutation(N) % CQ for _ in range(H)]).astype(np.int32)
    else:
        qlab = rng.integers(0, CQ - 1, (H, N)).astype(np.int32)   # cluster CQ-1 stays empty
    qperm, qcounts = O.stable_perm(qlab, CQ)
    if kind == "jumps":
        j = np.arange(N)
        scale = (1.0 + 0.6 * np.sin(j * 0.7) + 4.0 * ((j // 64) % 3 == 1)).astype(np.float32)
        for h in range(H):
            QU[h, qperm[h]] = (QU[h, qperm[h]].astype(np.float32) * scale[:, None]).astype(np.float16)
    if kind == "alternating_scale":
        scale = np.where(np.arange(N) % 2 == 1, 50.0, 0.02).astype(np.float32)
        for h in range(H):
            QU[h, qperm[h]] = (QU[h, qperm[h]].astype(np.float32) * scale[:, None]).astype(np.float16)
    _, cks = ops.centroid_finalize(g(ck2, dev))
    ns_t = torch.tensor(ns, dtype=torch.int32, device=dev)
    gl = ops.score(g(QU, dev), cks)
    u_split, r_split = ops.select_union(gl, g(sizes, dev), g(qperm, dev), g(qcounts, dev), ns_t)
    u_fused, r_fused = ops.score_select(g(QU, dev), cks, g(sizes, dev), g(qperm, dev),
                                        g(qcounts, dev), ns_t)
    assert torch.equal(u_fused, u_split) and torch.equal(r_fused, r_split)
    eu, er = O.select_union(c(gl), sizes, qperm, qcounts, ns)
    assert np.array_equal(c(u_fused), eu) and np.array_equal(c(r_fused), er)


def test_select_one_query_per_cluster_and_full_budget(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(9)
    H, N, CQ = 1, 512, 512
    gl = rng.normal(0, 1, (H, N, 2048)).astype(np.float16)
    sizes = rng.multinomial(N, np.ones(2048) / 2048)[None].astype(np.int32)
    qlab = rng.permutation(N)[None].astype(np.int32)
    qperm, qcounts = O.stable_perm(qlab, CQ)
    for ns in (1, N):
        ns_t = torch.tensor(ns, dtype=torch.int32, device=dev)
        unip, rowcnt = ops.select_union(g(gl, dev), g(sizes, dev), g(qperm, dev), g(qcounts, dev),
                                        ns_t)
        eu, er = O.select_union(gl, sizes, qperm, qcounts, ns)
        assert np.array_equal(c(unip), eu) and np.array_equal(c(rowcnt), er)


# ---------------------------------------------------------------------------
def test_kmeans_clear_clusters_exact(dev):
    """Well-separated data: labels agree exactly, so every output must be
    bit-identical to the oracle's."""
    from token2tile_amd import ops
    rng = np.random.default_rng(3)
    H, N, CQ, CK = 2, 6000, 64, 2048
    QU, cq0, _ = clustered(rng, H, N, 32, CQ)
    KU, ck0, _ = clustered(rng, H, N, 32, CK, spread=0.02)
    V = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    for pin in (0, 100):
        o = ops.kmm_run(g(QU, dev), g(KU, dev), g(V, dev), g(cq0, dev), g(ck0, dev), pin_tail=pin)
        e = O.kmeans_maintain(QU, KU, V, cq0, ck0, pin_tail=pin)
        for k in ("qlab", "qcounts", "qperm", "cq2", "klab", "kcounts", "kperm", "ck2", "V_sorted",
                  "sumv", "lam"):
            assert np.array_equal(c(o[k]), e[k]), (pin, k)


def test_kmeans_labels_near_ties_only_and_chained_exact(dev):
    """Random data: label disagreements only at near-ties; everything
    downstream of the GPU's labels is bit-exact."""
    from token2tile_amd import ops
    rng = np.random.default_rng(4)
    H, N, CQ, CK = 2, 5000, 96, 2048
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    KU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    cq0 = QU[:, rng.choice(N, CQ, replace=False)]
    ck0 = KU[:, rng.choice(N, CK, replace=False)]
    V = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    o = ops.kmm_run(g(QU, dev), g(KU, dev), g(V, dev), g(cq0, dev), g(ck0, dev))
    klab = c(o["klab"])
    d = O.assign_distances(KU, ck0)
    dmin = d.min(-1)
    mine = np.take_along_axis(d, klab[..., None].astype(np.int64), -1)[..., 0]
    assert np.all(mine - dmin <= 1e-4 * (1 + np.abs(dmin)))
    assert (klab != O.assign(KU, ck0)).mean() < 1e-3
    ks = O.key_side(KU, V, ck0, klab)
    for k in ("kcounts", "kperm", "ck2", "V_sorted", "sumv", "lam"):
        assert np.array_equal(c(o[k]), ks[k]), k
    qlab = c(o["qlab"])
    qperm, qcounts = O.stable_perm(qlab, CQ)
    assert np.array_equal(c(o["qperm"]), qperm) and np.array_equal(c(o["qcounts"]), qcounts)


def test_kmeans_labels_do_not_depend_on_label_buffer_contents(dev):
    """The assignment starts its running minimum from the label buffers' old
    contents (a guess plus a rounding bound); every output must be the same
    whatever those contents are: unset, the exact answer, wrong labels, or
    the higher index of duplicated centroids (exact ties -> lowest index)."""
    from token2tile_amd import ops
    rng = np.random.default_rng(41)
    H, N, CQ, CK = 2, 5000, 96, 2048
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    KU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    cq0 = QU[:, rng.choice(N, CQ, replace=False)].copy()
    ck0 = KU[:, rng.choice(N, CK, replace=False)].copy()
    ck0[:, 1500] = ck0[:, 7]                                 # exact ties: 7 must win
    cq0[:, 90] = cq0[:, 3]
    V = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    args = [g(a, dev) for a in (QU, KU, V, cq0, ck0)]

    def run(qlab0, klab0):
        out = {"qlab": g(qlab0.astype(np.int32), dev), "klab": g(klab0.astype(np.int32), dev)}
        o = ops.kmm_run(*args, out=out)
        return {k_: c(v_) for k_, v_ in o.items() if v_ is not None}

    base = run(np.full((H, N), -1), np.full((H, N), -1))
    exact_q, exact_k = base["qlab"], base["klab"]
    swap = lambda lab, a, b: np.where(lab == a, b, lab)   # noqa: E731
    for qg, kg in ((exact_q, exact_k),
                   ((exact_q + 1) % CQ, (exact_k + 5) % CK),
                   (swap(exact_q, 3, 90), swap(exact_k, 7, 1500)),
                   (rng.integers(-50, CQ + 50, (H, N)), rng.integers(-50, CK + 50, (H, N)))):
        o = run(qg, kg)
        for k_ in base:
            assert np.array_equal(o[k_], base[k_]), k_
    assert not np.any(exact_k == 1500) and np.any(exact_k == 7)


def test_vstats_reuse_paths(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(5)
    H, N = 2, 3000
    V = rng.normal(0, 3, (H, N, 128)).astype(np.float16)
    klab = rng.integers(0, 2000, (H, N)).astype(np.int32)
    kperm, kcounts = O.stable_perm(klab, 2048)
    eVs, esumv, elam, _ = O.v_statistics(V, kperm, kcounts)
    Vs, sumv, lam = ops.vstats_gather(g(V, dev), g(kperm, dev), g(kcounts, dev))
    assert np.array_equal(c(Vs), eVs) and np.array_equal(c(sumv), esumv)
    assert np.array_equal(c(lam), elam)
    sumv2, lam2 = ops.vstats(Vs, g(kcounts, dev))
    assert torch.equal(sumv2, sumv) and torch.equal(lam2, lam)
    Vb = g(V, dev).to(torch.bfloat16)
    Vsb, sumvb, lamb = ops.vstats_gather(Vb, g(kperm, dev), g(kcounts, dev))
    eVs2, esumv2, elam2, _ = O.v_statistics(c(Vb.float()), kperm, kcounts)
    assert np.array_equal(c(Vsb.float()), eVs2) and np.array_equal(c(sumvb), esumv2)


def test_init_helpers(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(6)
    x, cent, lab = clustered(rng, 2, 3000, 32, 100)
    got = c(ops.fast_assign_labels(g(x, dev), g(cent, dev)))
    assert np.array_equal(got, O.fast_assign(x, cent))
    new, counts = ops.det_centroid_update(g(x, dev), g(got, dev), g(cent, dev))
    en, ec = O.det_centroid_update(x, got, cent)
    assert np.array_equal(c(new), en) and np.array_equal(c(counts), ec)
    G = c(ops.gram(g(x, dev)))
    xd = x.astype(np.float64)
    assert np.allclose(G, np.einsum("hni,hnj->hij", xd, xd) / x.shape[1], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
def attn_case(rng, H=2, N=3000, CQ=24, density=0.1, empty_cluster=True):
    q = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    k = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    v = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    klab = rng.integers(0, 2048, (H, N)).astype(np.int32)
    kperm, kcounts = O.stable_perm(klab, 2048)
    qlab = rng.integers(0, CQ, (H, N)).astype(np.int32)
    if empty_cluster:
        qlab[qlab == 5] = 6
    qlab[:, :600] = 7                                        # one large cluster (> 128 rows)
    qperm, qcounts = O.stable_perm(qlab, CQ)
    sel = rng.random((H, CQ, 2048)) < density
    sel[:, 3] = False                                        # an empty union
    sel[:, 4] = True                                         # a full union
    unip = O.pack_bits(sel)
    kp = np.stack([k[h][kperm[h]] for h in range(H)])
    vp = np.stack([v[h][kperm[h]] for h in range(H)])
    return q, k, v, kperm, kcounts, qlab, qperm, qcounts, unip, kp, vp


def test_plan(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(7)
    q, k, v, kperm, kcounts, qlab, qperm, qcounts, unip, kp, vp = attn_case(rng)
    H, N, _ = q.shape
    CQ = qcounts.shape[1]
    plan = ops.tile_plan(g(qcounts, dev), g(kcounts, dev), g(unip, dev), N)
    pv = {k_: c(v_) for k_, v_ in ops.plan_views(plan, H, N, CQ).items()}
    assert np.array_equal(pv["k_off"][:, :2048], O.exclusive_scan(kcounts))
    uni = O.unpack_bits(unip)
    kvlen = np.where(qcounts > 0, (uni * kcounts[:, None, :]).sum(-1), 0)
    assert np.array_equal(pv["kvlen"], kvlen)
    qoff = O.exclusive_scan(qcounts)
    for h in range(H):
        nt = pv["ntask"][h]
        tasks = pv["tasks"][h, :nt]
        covered = np.zeros(N, dtype=int)
        for t, s, rows, _ in tasks:
            assert 1 <= rows <= 128 and qoff[h, t] <= s and s + rows <= qoff[h, t] + qcounts[h, t]
            covered[s:s + rows] += 1
        assert np.all(covered == 1)
        # whole waves of 32 queries: a cluster's tasks use ceil(n / 32) waves in
        # ceil(n / 128) tasks (only the last task of a cluster has a partial wave)
        for t in np.unique(tasks[:, 0]):
            rows = tasks[tasks[:, 0] == t, 2]
            n = qcounts[h, t]
            assert len(rows) == -(-n // 128)
            assert (-(-rows // 32)).sum() == -(-n // 32)
        # LPT by the cluster's largest task; a cluster's tasks are adjacent
        work = tasks[:, 3].astype(np.int64) * kvlen[h, tasks[:, 0]]
        assert np.all(np.diff(work) <= 0)
        assert np.all(tasks[:, 2] <= tasks[:, 3])
        first = {}
        for i, t in enumerate(tasks[:, 0]):
            first.setdefault(t, i)
            assert i - first[t] < -(-qcounts[h, t] // 128)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_tile_attention_exact(dev, dtype):
    from token2tile_amd import ops
    rng = np.random.default_rng(8)
    q, k, v, kperm, kcounts, qlab, qperm, qcounts, unip, kp, vp = attn_case(rng)
    H, N, _ = q.shape
    tq, tkp, tvp = (g(a, dev).to(dtype) for a in (q, kp, vp))
    plan = ops.tile_plan(g(qcounts, dev), g(kcounts, dev), g(unip, dev), N)
    ao, lse = ops.tile_attn_exact(tq, tkp, tvp, g(kcounts, dev), g(unip, dev), g(qperm, dev), plan)
    qf, kpf, vpf = (c(t.float()) for t in (tq, tkp, tvp))
    eo, el = O.tile_attention(qf, kpf, vpf, qcounts, kcounts, unip, qperm)
    got = c(ao.float())
    tol = 4e-3 if dtype == torch.float16 else 2e-2
    assert np.abs(got - eo).max() < tol
    fin = np.isfinite(el)
    assert np.array_equal(fin, np.isfinite(c(lse)))
    assert np.abs(c(lse)[fin] - el[fin]).max() < 2e-3
    assert np.all(got[~fin] == 0)


def test_exact_task_forms_and_tile_counts(dev):
    """Both task forms of the exact kernel at every tile count: query
    clusters of 1, 2, 3 and 4 waves (tasks of <= 3 waves stage their tiles
    from a producer wave, 4-wave tasks by all waves with a per-tile barrier),
    each with union lengths of 0, 2, 64, 66, 128, 130, 200 and 1000 keys
    (0, 1, 1, 2, 2, 3, 4 and 16 tiles), against the oracle, and the K/V
    gather through kperm bit-identical to the gathered kp / vp."""
    from token2tile_amd import ops
    rng = np.random.default_rng(31)
    H, N = 1, 4096
    sizes = (20, 50, 90, 128)
    nsel = (0, 1, 32, 33, 64, 65, 100, 500)          # key clusters of 2 rows each
    CQ = len(sizes) * len(nsel) + 1
    q = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    k = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    v = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    klab = rng.permutation(np.arange(N) // 2).astype(np.int32)[None]
    kperm, kcounts = O.stable_perm(klab, 2048)
    labs, sel = [], np.zeros((H, CQ, 2048), dtype=bool)
    t = 0
    for sz in sizes:
        for n in nsel:
            labs += [t] * sz
            sel[0, t, rng.choice(2048, n, replace=False)] = True
            t += 1
    labs += [t] * (N - len(labs))                    # the rest: one cluster, full union
    sel[0, t] = True
    qlab = rng.permutation(np.array(labs, dtype=np.int32))[None]
    qperm, qcounts = O.stable_perm(qlab, CQ)
    unip = O.pack_bits(sel)
    kp = np.stack([k[h][kperm[h]] for h in range(H)])
    vp = np.stack([v[h][kperm[h]] for h in range(H)])
    for dtype in (torch.float16, torch.bfloat16):
        tq, tk, tv, tkp, tvp = (g(a, dev).to(dtype) for a in (q, k, v, kp, vp))
        plan = ops.tile_plan(g(qcounts, dev), g(kcounts, dev), g(unip, dev), N)
        ao, lse = ops.tile_attn_exact(tq, tkp, tvp, g(kcounts, dev), g(unip, dev), g(qperm, dev),
                                      plan)
        qf, kpf, vpf = (c(t_.float()) for t_ in (tq, tkp, tvp))
        eo, el = O.tile_attention(qf, kpf, vpf, qcounts, kcounts, unip, qperm)
        got = c(ao.float())
        tol = 4e-3 if dtype == torch.float16 else 2e-2
        assert np.abs(got - eo).max() < tol
        fin = np.isfinite(el)
        assert np.array_equal(fin, np.isfinite(c(lse)))
        assert np.abs(c(lse)[fin] - el[fin]).max() < 2e-3
        assert np.all(got[~fin] == 0)
        args = (g(kcounts, dev), g(unip, dev), g(qperm, dev), plan)
        out_a, lse_a = torch.zeros_like(tq), torch.zeros(H, N, dtype=torch.float32, device=dev)
        out_b, lse_b = torch.zeros_like(tq), torch.zeros(H, N, dtype=torch.float32, device=dev)
        ops.tile_attn_exact_orig(tq, tkp, tvp, *args, out_a, lse_a)
        ops.tile_attn_exact_orig_gather_kv(tq, tk, tv, g(kperm, dev), *args, out_b, lse_b)
        assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)


def test_full_union_equals_sdpa(dev):
    from token2tile_amd import ops
    rng = np.random.default_rng(10)
    H, N, CQ = 2, 2048, 16
    q = torch.randn(H, N, 128, device=dev, dtype=torch.bfloat16)
    k = torch.randn(H, N, 128, device=dev, dtype=torch.bfloat16)
    v = torch.randn(H, N, 128, device=dev, dtype=torch.bfloat16)
    klab = rng.integers(0, 2048, (H, N)).astype(np.int32)
    kperm, kcounts = O.stable_perm(klab, 2048)
    qlab = rng.integers(0, CQ, (H, N)).astype(np.int32)
    qperm, qcounts = O.stable_perm(qlab, CQ)
    unip = O.pack_bits(np.ones((H, CQ, 2048), dtype=bool))
    kp = ops.fast_gather(k, g(kperm, dev))
    vp = ops.fast_gather(v, g(kperm, dev))
    plan = ops.tile_plan(g(qcounts, dev), g(kcounts, dev), g(unip, dev), N)
    ao, lse = ops.tile_attn_exact(q, kp, vp, g(kcounts, dev), g(unip, dev), g(qperm, dev), plan)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    ref_sorted = torch.stack([ref[h][g(qperm, dev)[h].long()] for h in range(H)])
    assert (ao.float() - ref_sorted).abs().max().item() < 2e-2


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_exact_orig_gather_equals_gathered(dev, dtype):
    """Exact attention with K read through kperm == the same kernel over
    kp = k[kperm], bit for bit (empty clusters and a partial last tile
    included in the case)."""
    from token2tile_amd import ops
    rng = np.random.default_rng(21)
    q, k, v, kperm, kcounts, qlab, qperm, qcounts, unip, kp, vp = attn_case(rng)
    H, N, _ = q.shape
    tq, tk, tkp, tvp = (g(a, dev).to(dtype) for a in (q, k, kp, vp))
    plan = ops.tile_plan(g(qcounts, dev), g(kcounts, dev), g(unip, dev), N)
    args = (g(kcounts, dev), g(unip, dev), g(qperm, dev), plan)
    out_a, lse_a = torch.zeros_like(tq), torch.zeros(H, N, dtype=torch.float32, device=dev)
    out_b, lse_b = torch.zeros_like(tq), torch.zeros(H, N, dtype=torch.float32, device=dev)
    ops.tile_attn_exact_orig(tq, tkp, tvp, *args, out_a, lse_a)
    ops.tile_attn_exact_orig_gather(tq, tk, g(kperm, dev), tvp, *args, out_b, lse_b)
    assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
    assert int(kcounts.min()) == 0  # the case holds empty key clusters
    # V read through kperm as well (original-order v, also as token-major views)
    out_c, lse_c = torch.zeros_like(tq), torch.zeros(H, N, dtype=torch.float32, device=dev)
    tv = g(v, dev).to(dtype)
    ops.tile_attn_exact_orig_gather_kv(tq, tk, tv, g(kperm, dev), *args, out_c, lse_c)
    assert torch.equal(out_a, out_c) and torch.equal(lse_a, lse_c)
    qm, km, vm = (t.transpose(0, 1).contiguous().transpose(0, 1) for t in (tq, tk, tv))
    om = torch.zeros(N, H, 128, dtype=dtype, device=dev)
    lse_d = torch.zeros(H, N, dtype=torch.float32, device=dev)
    ops.tile_attn_exact_orig_gather_kv(qm, km, vm, g(kperm, dev), *args, om.transpose(0, 1), lse_d)
    assert torch.equal(out_a, om.transpose(0, 1)) and torch.equal(lse_a, lse_d)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_tail_merge(dev, dtype):
    from token2tile_amd import ops
    rng = np.random.default_rng(11)
    H, N, CQ = 2, 1500, 12
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    cks = (rng.normal(0, 1, (H, 2048, 32)) * 0.3).astype(np.float16)
    sumv = rng.normal(0, 2, (H, 2048, 128)).astype(np.float16)
    kcounts = rng.integers(0, 5, (H, 2048)).astype(np.int32)
    qlab = rng.integers(0, CQ, (H, N)).astype(np.int32)
    qperm, qcounts = O.stable_perm(qlab, CQ)
    sel = rng.random((H, CQ, 2048)) < 0.2
    sel[:, 0] = False
    sel[:, 1] = True
    unip = O.pack_bits(sel)
    ao = torch.randn(H, N, 128, device=dev).to(dtype)
    lse = (torch.randn(H, N, device=dev) + 12.0)
    lse[:, :40] = -float("inf")
    lam = np.array([1.0, 2.5], dtype=np.float32)
    tw = torch.tensor(1.0, device=dev)
    out = ops.tail_merge(ao, lse, g(QU, dev), g(cks, dev), g(sumv, dev), g(kcounts, dev),
                         g(unip, dev), g(qlab, dev), g(qperm, dev), g(lam, dev), tw)
    eo = O.tail_merge(c(ao.float()).astype(np.float64), c(lse).astype(np.float64), QU, cks, sumv,
                      kcounts, unip, qlab, qperm, lam, 1.0)
    got = c(out.float())
    tol = 5e-3 if dtype == torch.float16 else 3e-2
    assert np.abs(got - eo).max() < tol * max(1.0, np.abs(eo).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_attention_tail_matches_oracle(dev, dtype):
    """run_planned (exact attention + residual + merge in one kernel) against
    the oracle's S5 followed by S6, including empty and full unions."""
    from token2tile_amd import ops
    rng = np.random.default_rng(12)
    q, k, v, kperm, kcounts, qlab, qperm, qcounts, unip, kp, vp = attn_case(rng, density=0.05)
    H, N, _ = q.shape
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    cks = (rng.normal(0, 1, (H, 2048, 32)) * 0.3).astype(np.float16)
    sumv = rng.normal(0, 1, (H, 2048, 128)).astype(np.float16)
    lam = np.array([1.0, 3.0], dtype=np.float32)
    tq, tkp, tvp = (g(a, dev).to(dtype) for a in (q, kp, vp))
    out = torch.empty_like(tq)
    plan = torch.empty(ops.plan_ints(H, N, qcounts.shape[1]), dtype=torch.int32, device=dev)
    ops.tile_attn_run_planned(tq, tkp, tvp, g(qcounts, dev), g(kcounts, dev), g(unip, dev),
                              g(QU, dev), g(cks, dev), g(sumv, dev), g(lam, dev), g(qlab, dev),
                              g(qperm, dev), torch.tensor(1.0, device=dev), out, plan, True)
    qf, kpf, vpf = (c(t.float()) for t in (tq, tkp, tvp))
    ao, lse = O.tile_attention(qf, kpf, vpf, qcounts, kcounts, unip, qperm)
    eo = O.tail_merge(ao, lse, QU, cks, sumv, kcounts, unip, qlab, qperm, lam, 1.0)
    got = c(out.float())
    tol = 5e-3 if dtype == torch.float16 else 2e-2
    assert np.abs(got - eo).max() < tol
    a, b = got.ravel().astype(np.float64), eo.ravel()
    assert a @ b / (np.linalg.norm(a) * np.linalg.norm(b)) > 0.9999


def test_wrappers_reject_mismatched_tensors(dev):
    """Every wrapper checks each tensor's shape, dtype and device before a
    kernel sees its pointer; each case below would otherwise be read or written
    out of bounds.  Nothing here launches a kernel."""
    from token2tile_amd import ops
    H, N, CQ = 2, 640, 8
    z = lambda *s, dt=torch.int32: torch.zeros(*s, dtype=dt, device=dev)  # noqa: E731
    q = z(H, N, 128, dt=torch.bfloat16)
    kcounts, qcounts, unip, qperm = z(H, 2048), z(H, CQ), z(H, CQ, 64), z(H, N)
    QU, cks = z(H, N, 32, dt=torch.float16), z(H, 2048, 32, dt=torch.float16)
    sumv, lam = z(H, 2048, 128, dt=torch.float16), z(H, dt=torch.float32)
    tailw = torch.tensor(1.0, device=dev)
    plan = z(ops.plan_ints(H, N, CQ))
    ns = z(1)
    bad = [
        lambda: ops.fast_gather(q, z(H, N - 1)),
        lambda: ops.fast_gather(q, qperm.to(torch.int64)),
        lambda: ops.fast_gather(q, qperm, out=torch.empty_like(q, dtype=torch.float16)),
        lambda: ops.tile_plan(qcounts, z(H, 1024), unip, N),
        lambda: ops.tile_plan(qcounts, kcounts, unip, N, plan=plan[:-1]),
        lambda: ops.tile_attn_exact(q, q[:, :-1].contiguous(), q, kcounts, unip, qperm, plan),
        lambda: ops.tile_attn_exact(q, q, q.to(torch.float16), kcounts, unip, qperm, plan),
        lambda: ops.tile_attn_exact(q, q, q, kcounts, unip, qperm.cpu(), plan),
        lambda: ops.tile_attn_run_planned(q, q, q, qcounts, kcounts, unip, QU, cks, sumv[:, :1024],
                                          lam, qperm, qperm, tailw, torch.empty_like(q), plan,
                                          True),
        lambda: ops.tile_attn_run_planned(q, q, q, qcounts, kcounts, unip, QU, cks, sumv, lam,
                                          qperm, qperm, tailw.double(), torch.empty_like(q),
                                          plan, True),
        lambda: ops.tail_merge(q, z(H, N, dt=torch.float32), QU, cks, sumv, kcounts, unip, qperm,
                               qperm, z(H + 1, dt=torch.float32), tailw),
        lambda: ops.centroid_tiles(cks, sumv, tiles=z(16, dt=torch.uint8)),
        lambda: ops.score_select(QU, cks, kcounts, z(H, N + 1), qcounts, ns),
        lambda: ops.score_select(QU, cks, kcounts, qperm, qcounts, z(2)),
        lambda: ops.score_select(QU, cks, kcounts, qperm, qcounts, ns,
                                 ws=z(1 << 20, dt=torch.float32)),
        lambda: ops.select_union(z(H, N, 2048, dt=torch.float16), kcounts, qperm, qcounts, ns,
                                 unip=z(H, CQ, 32)),
        lambda: ops.vstats(q, z(H, 2048, dt=torch.int64)),
        lambda: ops.vstats_gather(q, qperm, kcounts, lam=z(H, 2, dt=torch.float32)),
        lambda: ops.kmm_run(QU, QU, q[:, :-1].contiguous(), z(H, CQ, 32, dt=torch.float16),
                            cks),
        lambda: ops.fast_assign_labels(QU, z(H, 16, 16, dt=torch.float16)),
        lambda: ops.det_centroid_update(QU, z(H, N - 1), z(H, 16, 32, dt=torch.float16)),
        lambda: ops.project(q.transpose(1, 2), z(H, 128, 32, dt=torch.float16)),
        lambda: ops.union_or_last(z(H, CQ, 63)),
    ]
    for i, f in enumerate(bad):
        with pytest.raises(ValueError):
            f()
            pytest.fail(f"case {i} was accepted")
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("N,D", [(5003, 128), (777, 96), (64, 128)])
def test_gram_full_width(dev, dtype, N, D):
    """fp64 Gram on MFMA at the operator's width: the split partial sums add
    up to x^T x / N (products of fp16 values are exact in fp64)."""
    from token2tile_amd import ops
    rng = np.random.default_rng(N + D)
    x = rng.normal(0, 1, (3, N, D)).astype(np.float16)
    xt = g(x, dev)
    if dtype == "bf16":
        xt = xt.to(torch.bfloat16)
        x = xt.float().cpu().numpy().astype(np.float16)   # bf16 is rounded to fp16 first
    G = c(ops.gram(xt))
    xd = x.astype(np.float64)
    ref = np.einsum("hni,hnj->hij", xd, xd) / N
    assert np.allclose(G, ref, rtol=1e-12, atol=1e-12)
    assert np.array_equal(G, c(ops.gram(xt)))              # same result on every call


@pytest.mark.parametrize("vdtype", [None, torch.float16, torch.bfloat16])
def test_fused_update_vstats_matches_oracle(dev, vdtype):
    """The reference's fused_update_vstats surface: fp32 centroid and value
    means bit-exact with the oracle (both sum in row order), fp16 / v-dtype
    outputs unless return_fp32, out-of-range labels rejected."""
    from token2tile_amd import deploy_step
    rng = np.random.default_rng(22)
    H, N, C = 2, 3000, 100
    x = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    labels = rng.integers(0, C - 5, (H, N)).astype(np.int32)
    old = rng.normal(0, 1, (H, C, 32)).astype(np.float16)
    tv = None if vdtype is None else g(rng.normal(0, 2, (H, N, 128)).astype(np.float32), dev).to(vdtype)
    vf = None if tv is None else c(tv.float())
    ecent, ecounts, evmean = O.fused_update_vstats(x, labels, old, vf)
    cent, counts, vmean = deploy_step.fused_update_vstats(g(x, dev), g(labels, dev), g(old, dev),
                                                          tv, return_fp32=True)
    assert cent.dtype == torch.float32 and np.array_equal(c(cent), ecent)
    assert np.array_equal(c(counts), ecounts)
    if tv is None:
        assert vmean is None
    else:
        assert vmean.dtype == torch.float32 and np.array_equal(c(vmean), evmean)
    cent16, _, vmean16 = deploy_step.fused_update_vstats(g(x, dev), g(labels, dev).long(),
                                                         g(old, dev), tv)
    assert cent16.dtype == torch.float16 and torch.equal(cent16, cent.to(torch.float16))
    if tv is not None:
        assert vmean16.dtype == vdtype and torch.equal(vmean16, vmean.to(vdtype))
    bad = g(labels, dev).clone()
    bad[0, 0] = C
    with pytest.raises(ValueError, match="labels"):
        deploy_step.fused_update_vstats(g(x, dev), bad, g(old, dev))
