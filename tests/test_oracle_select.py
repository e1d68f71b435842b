"""Pins the oracle's selection + union (S4) independently of its formula.

* a brute-force pure-Python walk over the clusters sorted by (float value
  descending with +0 above -0, index ascending);
* an emulation of the reference CUDA kernel's histogram algorithm
  (oracle/ref_select_emulation.py) under arbitrary predicted windows;
* special cases: all scores tied, -0 vs +0, zero-size clusters at and
  around the crossing, ns = 1, ns = N, one query per cluster.
"""
import math

import numpy as np
import pytest

from oracle import t2t_oracle as O
from oracle.ref_select_emulation import kmain_row

C = 2048


def brute_select(row_f16, sizes, ns):
    items = []
    for c in range(C):
        v = float(row_f16[c])
        negzero = 1 if (v == 0.0 and math.copysign(1.0, v) < 0) else 0
        items.append((-v, negzero, c))
    items.sort()
    sel = np.zeros(C, dtype=bool)
    cum = 0
    for _, _, c in items:
        sel[c] = True
        cum += int(sizes[c])
        if cum >= ns:
            break
    return sel, cum


def random_case(rng, rows, N, kind="normal"):
    sizes = rng.multinomial(N, np.ones(C) / C).astype(np.int64)
    if kind == "zeros":
        sizes[rng.choice(C, 600, replace=False)] = 0
        sizes[0] += N - sizes.sum()
    if kind == "normal":
        g = rng.normal(0, 1.0, (rows, C)).astype(np.float16)
    elif kind == "coarse":       # many exact ties
        g = (np.round(rng.normal(0, 1.0, (rows, C)) * 4) / 4).astype(np.float16)
    elif kind == "tied":
        g = np.full((rows, C), 0.5, dtype=np.float16)
    elif kind == "signedzero":
        g = rng.choice(np.array([0.0, -0.0, 1.0, -1.0], dtype=np.float16), (rows, C))
    else:
        g = rng.normal(0, 1.0, (rows, C)).astype(np.float16)
    return g, sizes


@pytest.mark.parametrize("kind", ["normal", "coarse", "tied", "signedzero", "zeros"])
def test_select_rows_matches_brute_force(kind):
    rng = np.random.default_rng(7)
    N = 16384
    g, sizes = random_case(rng, 6, N, kind)
    for ns in (1, 37, 819, 5000, N):
        sel, rc = O.select_rows(g, sizes, ns)
        for i in range(g.shape[0]):
            bsel, brc = brute_select(g[i], sizes, ns)
            assert np.array_equal(sel[i], bsel), (kind, ns, i)
            assert rc[i] == brc


@pytest.mark.parametrize("kind", ["normal", "coarse", "tied", "signedzero", "zeros"])
def test_select_rows_matches_reference_kernel_algorithm(kind):
    rng = np.random.default_rng(11)
    N = 16384
    g, sizes = random_case(rng, 4, N, kind)
    keys = O.order_key(g).astype(np.int64)
    for ns in (1, 819, 4096):
        sel, rc = O.select_rows(g, sizes, ns)
        for i in range(g.shape[0]):
            # predicted windows: far above, far below, exact, random
            exact = int(np.sort(keys[i])[-max(1, ns * C // N)])
            for pred in (exact, exact - 300, exact + 300, 32000, -32000,
                         int(rng.integers(-32768, 32767))):
                esel, erc = kmain_row(keys[i], sizes, ns, pred)
                assert np.array_equal(esel, sel[i]), (kind, ns, i, pred)
                assert erc == rc[i], (kind, ns, i, pred)


def test_order_key_is_monotone_with_signed_zero():
    vals = np.array([-np.inf, -65504, -1.0, -6e-8, -0.0, 0.0, 6e-8, 1.0, 65504, np.inf],
                    dtype=np.float16)
    k = O.order_key(vals).astype(np.int64)
    assert np.all(np.diff(k) > 0)


def test_zero_size_clusters_around_crossing():
    sizes = np.zeros(C, dtype=np.int64)
    # descending values on clusters 0..9; sizes 3 except zero-size ones
    g = np.full((1, C), -10.0, dtype=np.float16)
    for c in range(10):
        g[0, c] = 10 - c
    sizes[[0, 2, 4, 6]] = 3       # clusters 1, 3, 5 are empty (before/after crossing)
    sizes[100] = 16384 - 12
    sel, rc = O.select_rows(g, sizes, 6)
    # order 0(3) 1(0) 2(3) -> crossing at cluster 2; empty cluster 1 before it is in,
    # empty cluster 3 after it is out
    assert sel[0, :4].tolist() == [True, True, True, False]
    assert rc[0] == 6
    sel, rc = O.select_rows(g, sizes, 7)
    assert sel[0, :6].tolist() == [True, True, True, True, True, False]
    assert rc[0] == 9


def test_union_over_segments_and_packing():
    rng = np.random.default_rng(3)
    H, N, CQ = 1, 4096, 16
    g = rng.normal(0, 1, (H, N, C)).astype(np.float16)
    kc = rng.multinomial(N, np.ones(C) / C)[None].astype(np.int32)
    qlab = rng.integers(0, CQ, (H, N)).astype(np.int32)
    qperm, qc = O.stable_perm(qlab, CQ)
    unip, rc = O.select_union(g, kc, qperm, qc, 100)
    sel, rc2 = O.select_rows(g[0], kc[0], 100)
    assert np.array_equal(rc[0], rc2)
    uni = O.unpack_bits(unip)
    for t in range(CQ):
        rows = np.nonzero(qlab[0] == t)[0]
        assert np.array_equal(uni[0, t], sel[rows].any(0))
    # LSB-first words: cluster c -> word c >> 5, bit c & 31
    c = 37
    one = np.zeros((1, C), dtype=bool)
    one[0, c] = True
    w = O.pack_bits(one).view(np.uint32)
    assert w[0, 1] == (1 << 5) and w.sum() == (1 << 5)


def test_budget_above_total_raises():
    g = np.zeros((1, C), dtype=np.float16)
    sizes = np.ones(C, dtype=np.int64)
    with pytest.raises(ValueError):
        O.select_rows(g, sizes, C + 1)
