"""Pins the oracle's k-means maintenance (S2) by independent checks:
brute-force argmin, numpy stable argsort / bincount, exact rational
arithmetic for the fixed-point query means, math.fsum for the fp32 sums,
and the closed form of lam / sumv."""
from fractions import Fraction

import numpy as np

from oracle import t2t_oracle as O


def test_assign_is_bruteforce_argmin_lowest_index():
    rng = np.random.default_rng(0)
    H, N, C, r = 2, 300, 40, 32
    x = rng.normal(0, 1, (H, N, r)).astype(np.float16)
    c = rng.normal(0, 1, (H, C, r)).astype(np.float16)
    c[0, 7] = c[0, 3]                     # exact duplicate centroid: tie -> 3
    lab = O.assign(x, c)
    for h in range(H):
        for i in range(N):
            d = [float(np.sum((x[h, i].astype(np.float64) - c[h, j].astype(np.float64)) ** 2))
                 - float(np.sum(x[h, i].astype(np.float64) ** 2)) for j in range(C)]
            best = min(d)
            first = next(j for j in range(C) if abs(d[j] - best) <= 1e-9)
            assert lab[h, i] == first
    assert not np.any(lab[0] == 7)


def test_pin_tail_forces_last_cluster():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (1, 100, 32)).astype(np.float16)
    c = rng.normal(0, 1, (1, 8, 32)).astype(np.float16)
    lab = O.assign(x, c, pin_tail=10)
    assert np.all(lab[0, 90:] == 7)


def test_stable_perm_and_counts():
    rng = np.random.default_rng(2)
    lab = rng.integers(0, 50, (2, 1000)).astype(np.int32)
    perm, counts = O.stable_perm(lab, 64)
    for h in range(2):
        assert np.array_equal(counts[h], np.bincount(lab[h], minlength=64))
        expect = sorted(range(1000), key=lambda i: (lab[h, i], i))
        assert perm[h].tolist() == expect


def test_fixed_point_query_mean_is_exact():
    rng = np.random.default_rng(3)
    H, N, C, r = 1, 500, 20, 32
    x = rng.normal(0, 2, (H, N, r)).astype(np.float16)
    lab = rng.integers(0, C - 2, (H, N)).astype(np.int32)   # clusters C-2, C-1 empty
    old = rng.normal(0, 1, (H, C, r)).astype(np.float16)
    new, counts = O.q_centroid_update(x, lab, old)
    for c in range(C):
        rows = np.nonzero(lab[0] == c)[0]
        if rows.size == 0:
            assert np.array_equal(new[0, c], old[0, c])
            continue
        for d in range(0, r, 7):
            S = 0
            for i in rows:
                v = Fraction(float(x[0, i, d])) * 32768
                fl = v.numerator // v.denominator
                rem = v - fl
                S += fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2) else 0)
            # fp32(S) / (32768 * fp32(n)) in fp32, then fp16
            want = np.float16(np.float32(np.float32(S) / np.float32(32768.0 * rows.size)))
            assert new[0, c, d] == want


def test_key_side_sums_sequential_fp32_and_means():
    rng = np.random.default_rng(4)
    H, N, CK, r = 1, 700, 30, 32
    KU = rng.normal(0, 1, (H, N, r)).astype(np.float16)
    V = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    ck0 = rng.normal(0, 1, (H, CK, r)).astype(np.float16)
    klab = rng.integers(0, CK - 1, (H, N)).astype(np.int32)
    ks = O.key_side(KU, V, ck0, klab)
    for c in range(CK):
        rows = np.nonzero(klab[0] == c)[0]       # stable order = ascending row
        if rows.size == 0:
            assert np.array_equal(ks["ck2"][0, c], ck0[0, c].astype(np.float32))
            continue
        acc = np.zeros(r, dtype=np.float32)
        for i in rows:
            acc = (acc + KU[0, i].astype(np.float32)).astype(np.float32)
        assert np.array_equal(ks["ck2"][0, c], (acc / np.float32(rows.size)).astype(np.float32))
        exact = np.array([np.float64(sum(Fraction(float(v)) for v in KU[0, rows, d]))
                          for d in range(r)])
        assert np.allclose(acc, exact, rtol=0, atol=1e-4)
    # V_sorted is V in kperm order; lam/sumv closed form
    assert np.array_equal(ks["V_sorted"][0], V[0][ks["kperm"][0]])
    _, _, lam, vsum = O.v_statistics(V, ks["kperm"], ks["kcounts"])
    assert lam[0] == max(np.float32(1.0), np.float32(np.abs(vsum).max() / 32768.0))
    big = V.copy()
    big[0, :, 0] = 60000
    _, sumv, lam2, vsum2 = O.v_statistics(big.astype(np.float16), ks["kperm"], ks["kcounts"])
    assert lam2[0] > 1 and np.abs(sumv.astype(np.float32)).max() <= 32768.0 * 1.001


def test_det_centroid_update_matches_exact_mean():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (1, 300, 32)).astype(np.float16)
    lab = rng.integers(0, 10, (1, 300)).astype(np.int32)
    old = np.zeros((1, 12, 32), dtype=np.float16)
    new, counts = O.det_centroid_update(x, lab, old)
    for c in range(10):
        rows = np.nonzero(lab[0] == c)[0]
        exact = x[0, rows].astype(np.float64).mean(0)
        assert np.allclose(new[0, c].astype(np.float64), exact, rtol=1e-3, atol=1e-3)
    assert np.all(new[0, 10:] == 0) and counts[0, 10:].sum() == 0


def test_fused_update_vstats_fp32_means():
    """The fp32 mean update (fused_update_vstats.py:72-115): centroid and
    value means within the fp32 rounding bound of the exact (fsum) means,
    empty clusters keep the old centroid and get a zero value mean, counts
    are the bincount."""
    import math
    rng = np.random.default_rng(21)
    H, N, C = 2, 700, 40
    x = rng.normal(0, 2, (H, N, 32)).astype(np.float16)
    v = rng.normal(0, 3, (H, N, 128)).astype(np.float16).astype(np.float32)
    labels = rng.integers(0, C - 3, (H, N)).astype(np.int32)     # clusters C-3.. stay empty
    old = rng.normal(0, 1, (H, C, 32)).astype(np.float16)
    cent, counts, vmean = O.fused_update_vstats(x, labels, old, v)
    eps = 2.0 ** -24
    for h in range(H):
        assert np.array_equal(counts[h], np.bincount(labels[h], minlength=C))
        for c in range(C):
            rows = np.flatnonzero(labels[h] == c)
            n = rows.size
            if n == 0:
                assert np.array_equal(cent[h, c], old[h, c].astype(np.float32))
                assert not vmean[h, c].any()
                continue
            for arr, got in ((x[h].astype(np.float64), cent[h, c]), (v[h].astype(np.float64),
                                                                      vmean[h, c])):
                exact = np.array([math.fsum(arr[rows, d]) for d in range(arr.shape[1])]) / n
                bound = (n + 2) * eps * np.abs(arr[rows]).sum(0) / n + 1e-30
                assert np.all(np.abs(got - exact) <= bound)
    # without v: the same centroids, no value means
    cent2, counts2, none = O.fused_update_vstats(x, labels, old)
    assert none is None and np.array_equal(cent2, cent) and np.array_equal(counts2, counts)
