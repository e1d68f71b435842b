"""Pins the oracle's projection (S1), centroid norms and the whole-call
compositions (full_call, reuse_call, kmeans_maintain) by independent checks:
exact rational dot products, math.fsum, dense attention at the full budget,
and the nearest-centroid / cluster-mean properties of the k-means passes."""
import math
from fractions import Fraction

import numpy as np
import torch

from oracle import t2t_oracle as O


def _exact_dot(a, b):
    return sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(a, b))


def _half_ulp16(v):
    v = abs(float(v))
    if v < 2.0 ** -14:
        return 2.0 ** -25
    return 2.0 ** (math.floor(math.log2(v)) - 11)


def test_project_is_rounded_exact_product():
    """QU[h, i, j] = fp16(sum_d x[h, i, d] * U[h, d, j]): within half an fp16
    ulp (plus the fp32 step) of the exact rational product; a transposed U
    or a dropped term fails."""
    rng = np.random.default_rng(40)
    x = rng.normal(0, 1, (2, 40, 128)).astype(np.float16)
    U = rng.normal(0, 0.2, (2, 128, 32)).astype(np.float16)
    QU = O.project(x, U)
    assert QU.shape == (2, 40, 32) and QU.dtype == np.float16
    for h, i, j in [(0, 0, 0), (0, 3, 31), (1, 39, 7), (1, 17, 16), (0, 25, 1)]:
        ex = float(_exact_dot(x[h, i], U[h, :, j]))
        assert abs(float(QU[h, i, j]) - ex) <= _half_ulp16(ex) * 1.001 + 2.0 ** -40, (h, i, j)


def test_centroid_norms_fsum_bound():
    rng = np.random.default_rng(41)
    c = rng.normal(0, 2, (2, 50, 32)).astype(np.float16)
    n = O.centroid_norms(c)
    assert n.dtype == np.float32
    c64 = c.astype(np.float64)
    for h in range(2):
        for j in range(50):
            ex = math.fsum(c64[h, j] ** 2)
            assert abs(float(n[h, j]) - ex) <= 34 * 2.0 ** -24 * ex
    # small integers: every partial sum is exact in fp32
    ci = np.arange(32, dtype=np.float16)[None, None, :]
    assert float(O.centroid_norms(ci)[0, 0]) == sum(i * i for i in range(32))


def _inputs(rng, H, N, spread=1.0):
    means = rng.normal(0, 1, (16, 128))
    comp = rng.integers(0, 16, N)
    base = means[comp] + rng.normal(0, 0.3, (N, 128))
    q = np.stack([base + rng.normal(0, spread * 0.1, (N, 128)) for _ in range(H)])
    k = np.stack([base + rng.normal(0, spread * 0.1, (N, 128)) for _ in range(H)])
    v = rng.normal(0, 1, (H, N, 128))
    return (q / math.sqrt(128)).astype(np.float16), k.astype(np.float16), v.astype(np.float16)


def _state(q, k, CQ, rng):
    Uq, Uk = O.online_u(q.astype(np.float32), k.astype(np.float32))
    Uq, Uk = Uq.astype(np.float16), Uk.astype(np.float16)
    H, N, _ = q.shape
    QU, KU = O.project(q, Uq), O.project(k, Uk)
    ck = np.stack([KU[h][np.sort(rng.permutation(N)[:2048] % N)] for h in range(H)])
    cq = np.stack([QU[h][np.sort(rng.permutation(N)[:CQ])] for h in range(H)])
    return dict(Uq=Uq, Uk=Uk, ck=ck, cq=cq)


def _dense(q, k, v):
    return torch.nn.functional.scaled_dot_product_attention(
        torch.tensor(q, dtype=torch.float64), torch.tensor(k, dtype=torch.float64),
        torch.tensor(v, dtype=torch.float64)).numpy()


def test_full_call_at_full_budget_is_dense_attention():
    """With ns = N every row selects every non-empty key cluster, the residual
    has no mass and the call is dense attention over all keys; the reuse call
    on the same inputs and snapshot gives the same output."""
    rng = np.random.default_rng(42)
    H, N, CQ = 2, 2304, 16
    q, k, v = _inputs(rng, H, N)
    state = _state(q, k, CQ, rng)
    out, st, new_state = O.full_call(q, k, v, state, N, CQ)
    ref = _dense(q, k, v)
    assert np.allclose(out, ref, atol=1e-9)
    assert np.all(st["rowcnt"] == N)
    # every union holds every non-empty cluster (empty ones sorted before a
    # row's crossing point are included too, which changes nothing)
    sel = O.unpack_bits(st["unip"])
    for h in range(H):
        live = st["qcounts"][h] > 0               # an empty query cluster has no union
        assert np.all(sel[h][live][:, st["kcounts"][h] > 0]) and not sel[h][~live].any()
    assert new_state["ck"].dtype == np.float16 and new_state["cq"] is st["cq2"]
    again = O.reuse_call(q, k, v, st)
    assert np.allclose(again, out, atol=1e-12)


def test_full_call_small_budget_properties():
    """At a small budget: each row's selected key count covers ns, the output
    stays close to dense (clustered inputs), a reuse on the same inputs repeats
    the full call, and pin_tail routes the last rows to cluster C-1, which
    every union then holds."""
    rng = np.random.default_rng(43)
    H, N, CQ, ns, pin = 1, 2304, 16, 300, 64
    q, k, v = _inputs(rng, H, N)
    state = _state(q, k, CQ, rng)
    out, st, _ = O.full_call(q, k, v, state, ns, CQ, pin_tail=pin)
    assert np.all(st["rowcnt"] >= ns)
    assert np.all(st["klab"][:, N - pin:] == 2047)
    assert np.all(O.unpack_bits(st["unip"])[..., 2047])
    ref = _dense(q, k, v)
    cos = (out * ref).sum(-1) / np.linalg.norm(out, axis=-1) / np.linalg.norm(ref, axis=-1)
    assert cos.min() > 0.95
    assert np.allclose(O.reuse_call(q, k, v, st), out, atol=1e-12)


def test_kmeans_maintain_nearest_and_mean_properties():
    """Each label is the nearest centroid of the pass's centroids (brute
    force, exact rationals, ties to the lowest index) and each new query
    centroid is the cluster mean to within the fixed-point and fp16
    rounding; qperm groups rows by label in row order."""
    rng = np.random.default_rng(44)
    H, N, CQ, CK, r = 1, 400, 6, 2048, 32
    QU = rng.normal(0, 1, (H, N, r)).astype(np.float16)
    KU = rng.normal(0, 1, (H, N, r)).astype(np.float16)
    V = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    cq0 = QU[:, :CQ].copy()
    ck0 = rng.normal(0, 1, (H, CK, r)).astype(np.float16)
    km = O.kmeans_maintain(QU, KU, V, cq0, ck0)

    def nearest(x, cents):
        xs = [Fraction(float(t)) for t in x]
        d = [sum((a - Fraction(float(b))) ** 2 for a, b in zip(xs, c)) for c in cents]
        return d.index(min(d))

    for i in range(0, N, 7):
        assert km["qlab1"][0, i] == nearest(QU[0, i], cq0[0])
        assert km["qlab"][0, i] == nearest(QU[0, i], km["cq1"][0])
    for i in range(0, N, 50):
        assert km["klab"][0, i] == nearest(KU[0, i], ck0[0])
    for lab, cen in ((km["qlab1"], km["cq1"]), (km["qlab"], km["cq2"])):
        for c in range(CQ):
            rows = np.flatnonzero(lab[0] == c)
            if rows.size:
                m = QU[0, rows].astype(np.float64).mean(0)
                tol = np.array([_half_ulp16(t) for t in m]) * 1.01 + 2.0 ** -15
                assert np.all(np.abs(cen[0, c].astype(np.float64) - m) <= tol)
    expect = sorted(range(N), key=lambda i: (km["qlab"][0, i], i))
    assert km["qperm"][0].tolist() == expect
    assert np.array_equal(km["qcounts"][0], np.bincount(km["qlab"][0], minlength=CQ))
