"""CPU restatement of the Token2Tile attention call (the parity oracle).

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline).

Every function restates one stage of the reference operator
(``/root/reference/token2tile/operator``) in numpy, cites the reference lines
it follows, and says how the restatement is pinned (the checks in
``tests/test_oracle_*.py``).  Arrays are numpy; heads are the leading axis.

Stage names follow the operator: projection (S1), k-means maintenance (S2),
scoring (S3), selection + union (S4), exact tile attention (S5), residual +
merge (S6), reuse (S7), projection fit (S0).

Conventions
-----------
* fp16 values are ``np.float16`` arrays; fp32 arithmetic is done on
  ``np.float32`` arrays with explicit sequential loops where the reference's
  summation order is fixed (per-cluster sums), so the results are bit-exact
  for those stages.
* Where the reference's arithmetic order is hardware-defined (an MMA dot
  product), the oracle computes the exact (fp64) value and the tests compare
  with a stated tolerance.
"""
from __future__ import annotations

import math

import numpy as np

C_KEYS = 2048          # key clusters (fixed by the reference kernels)
HEAD_DIM = 128
LN2 = 0.6931471805599453


# ---------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------

def f16(x):
    """Round to fp16 (round-to-nearest-even), as a float16 array."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def order_key(gl):
    """fp16 score -> int16 key that orders like the value, with -0 < +0.

    select_union/src/kernel.cu:56-74,160 (XFORM): u ^= ((u >> 15) & 1) * 0x7FFF.
    """
    u = np.ascontiguousarray(gl, dtype=np.float16).view(np.uint16).astype(np.uint32)
    u = u ^ (((u >> 15) & 1) * 0x7FFF)
    return u.astype(np.uint16).view(np.int16)


def exclusive_scan(x, axis=-1):
    c = np.cumsum(x, axis=axis, dtype=np.int64)
    return (c - x).astype(np.int64)


def stable_perm(labels, C):
    """Stable counting-sort permutation: sorted position -> original row.

    kmeans_maintain/src/kernels.cu:266-371 (hist/col_total/prefix/col_offset/
    scatter): rows of a cluster keep their original order.
    """
    H, N = labels.shape
    perm = np.argsort(labels, axis=1, kind="stable").astype(np.int32)
    counts = np.stack([np.bincount(labels[h], minlength=C)[:C] for h in range(H)]).astype(np.int32)
    return perm, counts


def pack_bits(sel):
    """bool [..., 2048] -> LSB-first int32 words [..., 64]: word c>>5, bit c&31.

    select_union/src/kernel.cu:447-488 (k_pack_partials).
    """
    s = sel.reshape(sel.shape[:-1] + (sel.shape[-1] // 32, 32)).astype(np.uint64)
    w = (s << np.arange(32, dtype=np.uint64)).sum(-1).astype(np.uint32)
    return w.view(np.int32)


def unpack_bits(words, C=C_KEYS):
    w = np.ascontiguousarray(words).view(np.uint32).astype(np.uint64)
    bits = (w[..., None] >> np.arange(32, dtype=np.uint64)) & 1
    return bits.reshape(words.shape[:-1] + (C,)).astype(bool)


# ---------------------------------------------------------------------------
# S0: projection fit
# ---------------------------------------------------------------------------

def online_u(qf, kf, r=32):
    """Matched rank-r projections Uq, Uk [H, D, r] (fp32).

    deploy_step.py:122-149 (per-head fp64 Gram, eigh with eigenvalues clamped
    at 1e-8, symmetric square root / inverse square root, SVD of Rq^T Rk).
    Pinned by the Eckart-Young invariants (tests/test_oracle_fit.py): the
    rank-r product equals the best rank-r approximation of Q K^T in the
    whitened metric, and Uq^T Mq Uq = diag(S_r) = Uk^T Mk Uk.
    """
    qf = np.asarray(qf, dtype=np.float64)
    kf = np.asarray(kf, dtype=np.float64)
    for name, t in (("q", qf), ("k", kf)):
        if not np.isfinite(t).all():
            raise RuntimeError(f"online_u: non-finite {name} input")
    Uqs, Uks = [], []
    for h in range(qf.shape[0]):
        q, k = qf[h], kf[h]
        Mq = q.T @ q / q.shape[0]
        Mk = k.T @ k / k.shape[0]
        eq, Vq = np.linalg.eigh(Mq)
        ek, Vk = np.linalg.eigh(Mk)
        eq = np.maximum(eq, 1e-8)
        ek = np.maximum(ek, 1e-8)
        Rq = (Vq * np.sqrt(eq)) @ Vq.T
        Rk = (Vk * np.sqrt(ek)) @ Vk.T
        Rqi = (Vq / np.sqrt(eq)) @ Vq.T
        Rki = (Vk / np.sqrt(ek)) @ Vk.T
        U, S, Vh = np.linalg.svd(Rq.T @ Rk)
        sr = np.sqrt(S[:r])
        Uqs.append((Rqi.T @ U[:, :r] * sr).astype(np.float32))
        Uks.append((Rki @ Vh[:r].T * sr).astype(np.float32))
    return np.stack(Uqs), np.stack(Uks)


# ---------------------------------------------------------------------------
# S1 / S3: projections and scores (MMA products: exact value, then rounding)
# ---------------------------------------------------------------------------

def project(x, U):
    """QU = fp16(x @ U) with fp32 accumulation (deploy_step.py:321-324).

    The oracle forms the exact product in fp64 and rounds once to fp16; the
    GPU rounds an fp32 accumulation, so the two agree to 1 fp16 ulp.
    """
    x = np.asarray(x, dtype=np.float64)
    U = np.asarray(U, dtype=np.float64)
    return (x @ U).astype(np.float32).astype(np.float16)


def scale_centroids(ck2, scale=1.0 / math.sqrt(HEAD_DIM)):
    """state['ck'] = fp16(ck2); cks = fp16(fp32(ck2 * fp32(scale))).

    deploy_step.py:389,393 (torch multiplies an fp32 tensor by a Python
    scalar in fp32, then casts to fp16).  Pinned bit for bit against torch-CPU
    in tests/test_oracle_init.py.
    """
    ck2 = np.asarray(ck2, dtype=np.float32)
    ck16 = ck2.astype(np.float16)
    cks = (ck2 * np.float32(scale)).astype(np.float32).astype(np.float16)
    return ck16, cks


def scores(QU, cks):
    """gl = fp16(QU @ cks^T), [H, N, 2048] (deploy_step.py:394)."""
    a = np.asarray(QU, dtype=np.float64)
    b = np.asarray(cks, dtype=np.float64)
    return np.matmul(a, np.swapaxes(b, 1, 2)).astype(np.float32).astype(np.float16)


# ---------------------------------------------------------------------------
# S2: k-means maintenance
# ---------------------------------------------------------------------------

def centroid_norms(c):
    """||c||^2 in fp32, summed sequentially over the 32 dims.

    kmeans_maintain/src/kernels.cu:85-98 (prep_cen_kernel).  Each square of an
    fp16 value is exact in fp32, so fused and unfused multiply-add agree.
    """
    c = np.asarray(c, dtype=np.float16).astype(np.float32)
    s = np.zeros(c.shape[:-1], dtype=np.float32)
    for d in range(c.shape[-1]):
        s = (s + c[..., d] * c[..., d]).astype(np.float32)
    return s


def assign_distances(x, c):
    """d[i, c] = ||c||^2 + sum_d x_d * (-2 c_d), exact (fp64) cross term.

    kmeans_maintain/src/kernels.cu:104-257: the MMA accumulates the cross term
    in fp32 starting from the fp32 norm; the oracle evaluates the same
    expression exactly, so labels agree except at near-ties.
    """
    cn = centroid_norms(c).astype(np.float64)
    xx = np.asarray(x, dtype=np.float16).astype(np.float64)
    cc = np.asarray(c, dtype=np.float16).astype(np.float64)
    return cn[:, None, :] + np.matmul(xx, np.swapaxes(-2.0 * cc, 1, 2))


def assign(x, c, pin_tail=0):
    """argmin_c with ties to the lowest index; rows >= N - pin_tail -> C-1.

    kmeans_maintain/src/kernels.cu:229-253 (argmin with lowest-index ties,
    PIN_TAIL override) and :855-864 (pin_begin = N - pin_tail, label CK-1).
    """
    d = assign_distances(x, c)
    lab = np.argmin(d, axis=-1).astype(np.int32)   # first minimum = lowest index
    if pin_tail > 0:
        lab[:, lab.shape[1] - pin_tail:] = c.shape[1] - 1
    return lab


def q_centroid_update(x, labels, old):
    """Fixed-point query-cluster means.

    kmeans_maintain/src/kernels.cu:538-616 (qsum_kernel, qreduce_kernel):
    S = sum over the cluster of rne(fp32(x) * 32768) as an integer,
    mean = fp16(fp32(S) / (32768 * fp32(n))); an empty cluster keeps ``old``.
    Returns (new fp16 [H, C, r], counts int32 [H, C]).
    """
    x = np.asarray(x, dtype=np.float16)
    H, N, r = x.shape
    C = old.shape[1]
    xi = np.rint(x.astype(np.float32) * np.float32(32768.0)).astype(np.int64)
    out = np.empty((H, C, r), dtype=np.float16)
    counts = np.zeros((H, C), dtype=np.int32)
    for h in range(H):
        S = np.zeros((C, r), dtype=np.int64)
        np.add.at(S, labels[h], xi[h])
        n = np.bincount(labels[h], minlength=C)[:C]
        counts[h] = n
        with np.errstate(invalid="ignore", divide="ignore"):    # empty clusters: replaced below
            mean = S.astype(np.float32) / (np.float32(32768.0) * n.astype(np.float32))[:, None]
            mean = mean.astype(np.float32).astype(np.float16)
        out[h] = np.where((n > 0)[:, None], mean, old[h])
    return out, counts


def _segment_sums_sequential(x, perm, counts):
    """fp32 sums of x rows per cluster, accumulated in perm order.

    kmeans_maintain/src/kernels.cu:374-429 (gather_kernel: one owner per
    cluster, rows in sorted order, fp32 adds).  The vector loop runs position
    p of every cluster at once, which keeps each cluster's order sequential.
    """
    C = counts.shape[0]
    base = exclusive_scan(counts)
    acc = np.zeros((C, x.shape[-1]), dtype=np.float32)
    xf = x.astype(np.float32)
    maxc = int(counts.max()) if C else 0
    for p in range(maxc):
        live = np.nonzero(counts > p)[0]
        rows = perm[base[live] + p]
        acc[live] = (acc[live] + xf[rows]).astype(np.float32)
    return acc


def v_statistics(V, kperm, kcounts):
    """V_sorted = V[kperm]; vsum in sorted order (fp32); lam; sumv fp16.

    kmeans_maintain/src/kernels.cu:374-429 (V part of gather_kernel),
    :481-531 (gather_v_permute_kernel, reuse calls), :649-692 (vred/vscale):
    lam = max(1, max|vsum| / 32768) per head; sumv = fp16(vsum * (1 / lam)).
    Returns (V_sorted [H,N,128] (input dtype), sumv fp16 [H,C,128],
    lam fp32 [H], vsum fp32 [H,C,128]).
    """
    H, N, D = V.shape
    C = kcounts.shape[1]
    V_sorted = np.stack([V[h][kperm[h]] for h in range(H)])
    vsum = np.stack([_segment_sums_sequential(V[h], kperm[h], kcounts[h]) for h in range(H)])
    lam = np.maximum(np.float32(1.0), np.abs(vsum).reshape(H, -1).max(axis=1) / np.float32(32768.0))
    lam = lam.astype(np.float32)
    inv = (np.float32(1.0) / lam).astype(np.float32)
    sumv = (vsum * inv[:, None, None]).astype(np.float32).astype(np.float16)
    return V_sorted, sumv, lam, vsum


def kmeans_maintain(QU, KU, V, cq0, ck0, pin_tail=0):
    """One warm-started k-means update: two query passes, one key pass.

    kmeans_maintain/src/kernels.cu:787-876 (kmeans_maintain_launch).
    Returns a dict with qlab, cq2, klab, ck2 (fp32), qcounts, qperm, kcounts,
    kperm, V_sorted, sumv, lam, plus the intermediates qlab1 and cq1.
    """
    H, N, _ = QU.shape
    CQ, CK = cq0.shape[1], ck0.shape[1]
    if not (0 <= pin_tail <= N):
        raise ValueError("pin_tail must be in [0, N]")
    qlab1 = assign(QU, cq0)
    cq1, _ = q_centroid_update(QU, qlab1, cq0)
    qlab = assign(QU, cq1)
    cq2, qcounts = q_centroid_update(QU, qlab, cq1)
    qperm, qcounts2 = stable_perm(qlab, CQ)
    assert np.array_equal(qcounts, qcounts2)
    klab = assign(KU, ck0, pin_tail=pin_tail)
    return dict(qlab1=qlab1, cq1=cq1, qlab=qlab, cq2=cq2, qcounts=qcounts, qperm=qperm,
                klab=klab, **key_side(KU, V, ck0, klab))


def key_side(KU, V, ck0, klab):
    """Key grouping, fp32 key centroids and value statistics from labels.

    kmeans_maintain/src/kernels.cu:865-875: counts, stable kperm, per-cluster
    fp32 sums of KU in kperm order, ck2 = sum / n (empty -> fp32(ck0)),
    then the value statistics of ``v_statistics``.
    """
    H = KU.shape[0]
    CK = ck0.shape[1]
    kperm, kcounts = stable_perm(klab, CK)
    ck2 = np.empty((H, CK, KU.shape[2]), dtype=np.float32)
    for h in range(H):
        ks = _segment_sums_sequential(KU[h], kperm[h], kcounts[h])
        n = kcounts[h].astype(np.float32)[:, None]
        with np.errstate(invalid="ignore", divide="ignore"):
            mean = (ks / n).astype(np.float32)
        ck2[h] = np.where(kcounts[h][:, None] > 0, mean, ck0[h].astype(np.float32))
    V_sorted, sumv, lam, _ = v_statistics(V, kperm, kcounts)
    return dict(kcounts=kcounts, kperm=kperm, ck2=ck2, V_sorted=V_sorted, sumv=sumv, lam=lam)


# ---------------------------------------------------------------------------
# S4: per-query selection and query-cluster union
# ---------------------------------------------------------------------------

def select_rows(gl_rows, sizes, ns):
    """Selection of each row: the shortest prefix of clusters, ordered by
    (score key descending, cluster index ascending), whose sizes sum to >= ns.

    select_union/src/kernel.cu:190-412 (k_main).  Returns (sel bool [R, C],
    rowcnt int32 [R]).  Zero-size clusters before the crossing cluster are in
    the prefix; those after it are not.  Requires ns <= sum(sizes).
    Pinned against a brute-force Python sort and against an emulation of the
    reference kernel's histogram algorithm (tests/test_oracle_select.py).
    """
    key = order_key(gl_rows).astype(np.int32)
    R, C = key.shape
    comp = ((32767 - key).astype(np.int64) << 12) | np.arange(C, dtype=np.int64)[None, :]
    order = np.argsort(comp, axis=1, kind="stable")
    sz = np.asarray(sizes, dtype=np.int64)[order]
    cum = np.cumsum(sz, axis=1)
    if (cum[:, -1] < ns).any():
        raise ValueError("budget ns exceeds the number of keys")
    cross = np.argmax(cum >= ns, axis=1)            # first position reaching ns
    take = np.arange(C)[None, :] <= cross[:, None]
    sel = np.zeros((R, C), dtype=bool)
    np.put_along_axis(sel, order, take, axis=1)
    rowcnt = cum[np.arange(R), cross].astype(np.int32)
    return sel, rowcnt


def select_union(gl, kcounts, qperm, qcounts, ns):
    """Union of the selections of each query cluster, packed, plus rowcnt.

    select_union/src/kernel.cu:76-97 (k_offsets: rows of cluster t are
    qperm[off[t] : off[t] + qcounts[t]]), :190-412 (k_main), :447-488
    (k_pack_partials).  Returns (unip int32 [H, CQ, 64], rowcnt int32 [H, N]).
    rowcnt is written at the original row index; rows outside every segment
    keep 0 here.
    """
    H, N, C = gl.shape
    CQ = qcounts.shape[1]
    unip = np.zeros((H, CQ, C // 32), dtype=np.int32)
    rowcnt = np.zeros((H, N), dtype=np.int32)
    for h in range(H):
        sel, rc = select_rows(gl[h], kcounts[h], ns)
        rowcnt[h] = rc
        off = exclusive_scan(qcounts[h])
        uni = np.zeros((CQ, C), dtype=bool)
        for t in range(CQ):
            rows = qperm[h, off[t]: off[t] + qcounts[h, t]]
            if rows.size:
                uni[t] = sel[rows].any(axis=0)
        unip[h] = pack_bits(uni)
    return unip, rowcnt


def or_pin_tail(unip, C=C_KEYS):
    """Every query cluster executes the reserved last key cluster.

    deploy_step.py:444-448.  Pinned in tests/test_oracle_init.py against the
    reference's byte-view formula and the one-bit-changed invariant.
    """
    out = unip.copy().view(np.uint32)
    out[..., (C - 1) >> 5] |= np.uint32(1) << np.uint32((C - 1) & 31)
    return out.view(np.int32)


# ---------------------------------------------------------------------------
# S5: exact attention over the union
# ---------------------------------------------------------------------------

def kv_rows_of_union(uni_row, k_off):
    """Cluster-ordered key rows of one union, clusters in ascending index.

    tile_attn/src/kernel.cu:279-299 (k_off = exclusive scan of the key
    cluster sizes) and :868-920 (runs of selected, non-empty clusters in
    ascending cluster order).
    """
    cl = np.nonzero(uni_row)[0]
    if cl.size == 0:
        return np.zeros(0, dtype=np.int64)
    return np.concatenate([np.arange(k_off[c], k_off[c + 1]) for c in cl])


def tile_attention(q, kp, vp, qcounts, kcounts, unip, qperm, scale=1.0 / math.sqrt(HEAD_DIM),
                   heads=None, clusters=None):
    """Exact attention of every sorted query over its cluster's union.

    tile_attn/src/kernel.cu:820-1096 (attn_kernel): query j of the sorted
    order (original row qperm[j]) attends to the concatenated union rows of
    kp/vp; output and lse stay in sorted order; lse is log2 of the softmax
    denominator; an empty union gives o = 0 and lse = -inf (:946-956).
    Computed in fp64.  Pinned by: an all-ones union equals dense attention
    (torch SDPA) and a single-cluster union equals a hand-sliced softmax.
    Returns (out fp64 [H, N, D] sorted order, lse fp64 [H, N]).
    ``heads`` / ``clusters`` restrict the work to those heads and query
    clusters (the other rows stay 0 / -inf), so a caller can split one call
    over processes.
    """
    H, N, D = q.shape
    CQ = qcounts.shape[1]
    out = np.zeros((H, N, D), dtype=np.float64)
    lse = np.full((H, N), -np.inf, dtype=np.float64)
    uni = unpack_bits(unip)
    for h in (range(H) if heads is None else heads):
        k_off = np.concatenate([[0], np.cumsum(kcounts[h])])
        qoff = exclusive_scan(qcounts[h])
        kh = kp[h].astype(np.float64)
        vh = vp[h].astype(np.float64)
        for t in (range(CQ) if clusters is None else clusters):
            n = int(qcounts[h, t])
            if n == 0:
                continue
            rows = kv_rows_of_union(uni[h, t], k_off)
            if rows.size == 0:
                continue
            js = np.arange(qoff[t], qoff[t] + n)
            qq = q[h][qperm[h, js]].astype(np.float64)
            s = (qq @ kh[rows].T) * scale
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            out[h, js] = (p @ vh[rows]) / l
            lse[h, js] = (m[:, 0] + np.log(l[:, 0])) / LN2
    return out, lse


# ---------------------------------------------------------------------------
# S6: centroid residual over the unselected clusters, and the merge
# ---------------------------------------------------------------------------

def tail_merge(attn_out, attn_lse, QU, cks, sumv, kcounts, unip, qlab, qperm, lam, tailw=1.0,
               heads=None, rows=None):
    """Per-query residual over the clusters outside its union, merged under
    one softmax with the exact part; written at the original row.

    tile_attn/src/kernel.cu:1172-1450 (tail_wgmma_kernel): s_c =
    fp16(QU . cks_c); p_c = exp(s_c - m); phi = sum p_c * n_c; O = sum
    fp16(p_c) * sumv_c over c outside the union; le = lse * ln2;
    ex = exp(le - M), st = exp(m - M) with M = max(le, m); if st*phi <=
    1e-6 * ex the exact output is kept, else out = (ex*o + st*tw*lam*O) / den
    with den = max(ex + st*phi*tw, 1e-12).  m is any finite shift (the
    result is shift invariant); the oracle uses max_c s_c + 2 like the
    reference.  Pinned by closed forms: empty union -> lam*O/phi; full union
    -> exact output; tw = 0 -> exact output (tests/test_oracle_attention.py).
    ``heads`` / ``rows`` (a slice of sorted positions) restrict the work; the
    other rows of the result stay 0.
    """
    H, N, D = attn_out.shape
    out = np.zeros((H, N, D), dtype=np.float64)
    uni = unpack_bits(unip)
    sl = slice(None) if rows is None else rows
    for h in (range(H) if heads is None else heads):
        cnt = kcounts[h].astype(np.float64)
        sv = sumv[h].astype(np.float64)
        orig = qperm[h][sl]
        s = scores(QU[h][orig][None], cks[h][None])[0].astype(np.float64)   # sorted order
        mask = uni[h][qlab[h][orig]]                       # in-union clusters
        m = s.max(axis=1) + 2.0
        p = np.where(mask, 0.0, np.exp(s - m[:, None]))
        phi = p @ cnt
        p16 = p.astype(np.float32).astype(np.float16).astype(np.float64)
        O = p16 @ sv
        le = attn_lse[h][sl] * LN2
        M = np.maximum(le, m)
        with np.errstate(invalid="ignore"):
            ex = np.exp(le - M)
            st = np.exp(m - M)
        ph = st * phi
        bad = ph <= 1e-6 * ex
        den = np.maximum(ex + ph * tailw, 1e-12)
        ao = attn_out[h][sl]
        merged = (ex / den)[:, None] * ao + (st * tailw * lam[h] / den)[:, None] * O
        res = np.where(bad[:, None], ao, merged)
        out[h, orig] = res
    return out


# ---------------------------------------------------------------------------
# init_state helpers (fast_assign and the deterministic centroid update)
# ---------------------------------------------------------------------------

def fast_assign(x, c):
    """Nearest centroid by ||x||^2 - 2 x.c + ||c||^2, ties to the lowest index.

    fast_assign.py:16-106.  The reference packs the cluster index into the
    low mantissa bits of the fp32 distance; the oracle uses the exact
    distance, so labels agree except where two distances are within the
    packing resolution.  Pinned against an exact-rational brute-force argmin
    with duplicated centroids (tests/test_oracle_init.py).
    """
    xx = np.asarray(x, dtype=np.float16).astype(np.float64)
    cc = np.asarray(c, dtype=np.float16).astype(np.float64)
    d = (xx * xx).sum(-1)[:, :, None] + (cc * cc).sum(-1)[:, None, :] - 2.0 * np.matmul(xx, np.swapaxes(cc, 1, 2))
    return np.argmin(d, axis=-1).astype(np.int32)


def det_centroid_update(x, labels, old):
    """int64 fixed-point (2^-20) centroid means; empty clusters keep ``old``.

    integrations/sglang/backend/t2t_attn.py:242-257 (_det_centroid_update):
    xi = round_half_even(x * 2^20); cent = (sum / 2^20) / n in fp64, cast to
    fp16 through fp32 (torch's double -> half conversion).  Pinned bit for bit
    against exact rational sums and torch-CPU's cast, with constructed
    rounding cases (tests/test_oracle_init.py).
    Returns (new fp16 [H, C, D], counts int32 [H, C]).
    """
    x = np.asarray(x, dtype=np.float16)
    H, N, D = x.shape
    C = old.shape[1]
    xi = np.rint(x.astype(np.float64) * 1048576.0).astype(np.int64)
    out = np.empty((H, C, D), dtype=np.float16)
    counts = np.zeros((H, C), dtype=np.int32)
    for h in range(H):
        S = np.zeros((C, D), dtype=np.int64)
        np.add.at(S, labels[h], xi[h])
        n = np.bincount(labels[h], minlength=C)[:C]
        counts[h] = n
        cent = (S.astype(np.float64) / 1048576.0) / np.maximum(n, 1)[:, None].astype(np.float64)
        cent = np.where((n > 0)[:, None], cent, old[h].astype(np.float64))
        out[h] = cent.astype(np.float32).astype(np.float16)
    return out, counts


def fused_update_vstats(x, labels, old, v=None):
    """fp32 centroid means and per-cluster value means.

    fused_update_vstats.py:72-115: per cluster, fp32 sums of the x rows (and
    v rows); new centroid = sum / n, an empty cluster keeps fp32(old); value
    mean = sum / max(n, 1).  The reference adds with fp32 atomics in no fixed
    order; this restatement adds in row order (the order of the stable
    cluster grouping), which is the order the HIP kernel uses.  Pinned in
    tests/test_oracle_kmeans.py against exact (math.fsum) means to the fp32
    rounding bound, and the empty-cluster rules.
    Returns (cent fp32 [H, C, D], counts int32 [H, C], vmean fp32 or None).
    """
    x = np.asarray(x, dtype=np.float16)
    H, N, D = x.shape
    C = old.shape[1]
    perm, counts = stable_perm(np.asarray(labels, dtype=np.int32), C)
    cent = np.empty((H, C, D), dtype=np.float32)
    vmean = None if v is None else np.empty((H, C, v.shape[2]), dtype=np.float32)
    for h in range(H):
        n = counts[h].astype(np.float32)[:, None]
        sk = _segment_sums_sequential(x[h], perm[h], counts[h])
        with np.errstate(invalid="ignore", divide="ignore"):
            mean = (sk / n).astype(np.float32)
        cent[h] = np.where(counts[h][:, None] > 0, mean, old[h].astype(np.float32))
        if v is not None:
            sv = _segment_sums_sequential(np.asarray(v[h], dtype=np.float32), perm[h], counts[h])
            vmean[h] = (sv / np.maximum(n, np.float32(1.0))).astype(np.float32)
    return cent, counts, vmean


# ---------------------------------------------------------------------------
# whole call
# ---------------------------------------------------------------------------

def full_call(q, k, v, state, ns, CQ, *, pin_tail=0, tailw=1.0):
    """One structure-rebuilding call of MaskedStepDeploy.step, on CPU.

    deploy_step.py:286-477 with snap is None: projections, k-means
    maintenance, scores, selection + union (+ pin-tail bit), key gather,
    exact attention, residual merge.  Returns (out fp64 [H, N, 128] in
    original order, structure dict, new state dict).
    """
    QU = project(q, state["Uq"])
    KU = project(k, state["Uk"])
    km = kmeans_maintain(QU, KU, v, state["cq"], state["ck"], pin_tail=pin_tail)
    ck16, cks = scale_centroids(km["ck2"])
    gl = scores(QU, cks)
    unip, rowcnt = select_union(gl, km["kcounts"], km["qperm"], km["qcounts"], ns)
    if pin_tail:
        unip = or_pin_tail(unip)
    kp = np.stack([k[h][km["kperm"][h]] for h in range(k.shape[0])])
    ao, lse = tile_attention(q, kp, km["V_sorted"], km["qcounts"], km["kcounts"], unip, km["qperm"])
    out = tail_merge(ao, lse, QU, cks, km["sumv"], km["kcounts"], unip, km["qlab"], km["qperm"],
                     km["lam"], tailw)
    struct = dict(km, QU=QU, KU=KU, cks=cks, gl=gl, unip=unip, rowcnt=rowcnt, kp=kp,
                  attn_out=ao, attn_lse=lse, Uq=state["Uq"])
    new_state = dict(state, ck=ck16, cq=km["cq2"])
    return out, struct, new_state


def reuse_call(q, k, v, snap, *, tailw=1.0):
    """One structure-reusing call (deploy_step.py:296-316,321-326,374-383):
    QU from the snapshot's Uq, K grouped through the stored kperm, value
    statistics recomputed from this call's V; everything else reused."""
    QU = project(q, snap["Uq"])
    kp = np.stack([k[h][snap["kperm"][h]] for h in range(k.shape[0])])
    V_sorted, sumv, lam, _ = v_statistics(v, snap["kperm"], snap["kcounts"])
    ao, lse = tile_attention(q, kp, V_sorted, snap["qcounts"], snap["kcounts"], snap["unip"], snap["qperm"])
    return tail_merge(ao, lse, QU, snap["cks"], sumv, snap["kcounts"], snap["unip"], snap["qlab"],
                      snap["qperm"], lam, tailw)
