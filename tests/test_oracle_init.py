"""Pins the oracle functions that define bit-exact GPU outputs but are not
covered by the stage tests: fast_assign (brute-force argmin), or_pin_tail
(the reference's byte-view formula, computed independently), scale_centroids
(torch-CPU fp32 scalar multiply and fp16 casts) and det_centroid_update
(exact rational fixed-point sums with round-half-even, fp64 division and
torch-CPU's fp64 -> fp16 conversion)."""
import math
from fractions import Fraction

import numpy as np
import torch

from oracle import t2t_oracle as O


def _brute_nearest(xrow, cent):
    """argmin_j ||x - c_j||^2 over exact rationals; ties to the lowest j."""
    xs = [Fraction(float(v)) for v in xrow]
    best, arg = None, -1
    for j in range(cent.shape[0]):
        d = sum((a - Fraction(float(b))) ** 2 for a, b in zip(xs, cent[j]))
        if best is None or d < best:
            best, arg = d, j
    return arg


def test_fast_assign_is_bruteforce_argmin_lowest_index():
    """fast_assign.py:16-106: nearest centroid, lowest index on ties."""
    rng = np.random.default_rng(31)
    H, N, C, D = 2, 120, 24, 32
    x = rng.normal(0, 1, (H, N, D)).astype(np.float16)
    c = rng.normal(0, 1, (H, C, D)).astype(np.float16)
    c[0, 11] = c[0, 4]                    # exact duplicate: the tie goes to 4
    c[1, 0] = c[1, 23]                    # duplicate of the last: the tie goes to 0
    x[0, :10] = c[0, 4]                   # rows sitting exactly on the duplicate
    x[1, :10] = c[1, 23]
    lab = O.fast_assign(x, c)
    assert lab.dtype == np.int32 and lab.shape == (H, N)
    for h in range(H):
        for i in range(N):
            assert lab[h, i] == _brute_nearest(x[h, i], c[h]), (h, i)
    assert not np.any(lab[0] == 11) and not np.any(lab[1] == 23)
    assert np.all(lab[0, :10] == 4) and np.all(lab[1, :10] == 0)


def test_fast_assign_norm_term_sign():
    """A centroid nearer in angle but much longer loses: a flipped sign of the
    ||c||^2 term, or a dropped ||c||^2, would pick it."""
    x = np.zeros((1, 1, 32), dtype=np.float16)
    x[0, 0, 0] = 1.0
    c = np.zeros((1, 3, 32), dtype=np.float16)
    c[0, 0, 0] = 8.0                      # dot 8, distance 49
    c[0, 1, 0] = 0.9                      # dot 0.9, distance 0.01
    c[0, 2, 1] = 0.5                      # dot 0, distance 1.25
    assert O.fast_assign(x, c)[0, 0] == 1


def test_or_pin_tail_sets_only_bit_31_of_word_63():
    """deploy_step.py:444-448 sets bit (C-1)&7 of byte (C-1)>>3 of each row's
    byte view. Restated independently on the words and on the bytes."""
    rng = np.random.default_rng(32)
    unip = rng.integers(-2**31, 2**31, (3, 5, 64), dtype=np.int64).astype(np.int32)
    unip[..., 63] &= 0x7FFFFFFF           # last bit clear everywhere
    unip[1, 2, 63] |= np.int32(-2**31)    # ... except one row where it is already set
    out = O.or_pin_tail(unip)
    assert out.dtype == np.int32 and out.shape == unip.shape
    assert np.array_equal(out[..., :63], unip[..., :63])
    w_in = unip[..., 63].astype(np.int64) & 0xFFFFFFFF
    w_out = out[..., 63].astype(np.int64) & 0xFFFFFFFF
    assert np.all(w_out == (w_in | (1 << 31)))
    # the reference's own byte-view formula, on a torch CPU tensor
    t = torch.from_numpy(unip.copy())
    t.view(torch.uint8).reshape(3, 5, -1)[:, :, 2047 >> 3] |= 1 << (2047 & 7)
    assert np.array_equal(t.numpy(), out)
    # idempotent; the input is not modified
    assert np.array_equal(O.or_pin_tail(out), out)
    assert not np.array_equal(out, unip)


def test_scale_centroids_matches_torch_cpu():
    """deploy_step.py:389,393: state['ck'] = ck2.to(fp16) and
    cks = (ck2 * (1/sqrt(128))).to(fp16), an fp32 tensor times a Python
    scalar, which torch evaluates in fp32."""
    rng = np.random.default_rng(33)
    ck2 = (rng.normal(0, 3, (2, 2048, 32)) * np.exp(rng.normal(0, 2, (2, 2048, 32)))).astype(np.float32)
    ck16, cks = O.scale_centroids(ck2)
    t = torch.from_numpy(ck2)
    want_ck = t.to(torch.float16).numpy()
    want_cks = (t * (1.0 / math.sqrt(128))).to(torch.float16).numpy()
    assert np.array_equal(ck16.view(np.uint16), want_ck.view(np.uint16))
    assert np.array_equal(cks.view(np.uint16), want_cks.view(np.uint16))
    # the order matters: casting to fp16 before the multiply gives other bits
    early = (t.to(torch.float16) * (1.0 / math.sqrt(128))).to(torch.float16).numpy()
    assert not np.array_equal(early.view(np.uint16), cks.view(np.uint16))


def _rne(fr):
    """Round a Fraction half to even."""
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2):
        fl += 1
    return fl


def _det_update_exact(x, labels, old):
    """t2t_attn.py:242-257 with exact arithmetic: S = sum rne(x * 2^20),
    mean = fl64(fl64(S / 2^20) / n), then torch-CPU's fp64 -> fp16 cast."""
    H, N, D = x.shape
    C = old.shape[1]
    out = np.empty((H, C, D), dtype=np.float64)
    for h in range(H):
        for c in range(C):
            rows = np.flatnonzero(labels[h] == c)
            for d in range(D):
                if rows.size == 0:
                    out[h, c, d] = float(old[h, c, d])
                    continue
                S = sum(_rne(Fraction(float(x[h, i, d])) * 2 ** 20) for i in rows)
                out[h, c, d] = (float(S) / 1048576.0) / float(rows.size)
    return torch.from_numpy(out).to(torch.float16).numpy()


def test_det_centroid_update_bit_exact():
    rng = np.random.default_rng(34)
    H, N, C, D = 2, 400, 14, 8
    x = rng.normal(0, 1.5, (H, N, D)).astype(np.float16)
    x[:, :40] = (rng.normal(0, 1, (H, 40, D)) * 2.0 ** -18).astype(np.float16)   # subnormal-scale rows
    labels = rng.integers(0, C - 2, (H, N)).astype(np.int32)    # last two clusters empty
    old = rng.normal(0, 1, (H, C, D)).astype(np.float16)
    new, counts = O.det_centroid_update(x, labels, old)
    want = _det_update_exact(x, labels, old)
    assert np.array_equal(new.view(np.uint16), want.view(np.uint16))
    assert np.array_equal(new[:, C - 2:], old[:, C - 2:])
    for h in range(H):
        assert np.array_equal(counts[h], np.bincount(labels[h], minlength=C))


def test_det_centroid_update_rounding_cases():
    """Constructed cases that a plausible slip fails:
    * x*2^20 = 0.5 and 1.5 round half to even (to 0 and 2): floor, or half
      away from zero, gives other sums;
    * a scale of 2^-16 in place of 2^-20 loses those sub-2^-16 values;
    * a mean just above an fp16 midpoint by less than half an fp32 ulp: the
      fp64 -> fp32 -> fp16 conversion torch does gives the even neighbour,
      a direct fp64 -> fp16 rounding gives the odd one."""
    D = 4
    # cluster 0: n = 64 rows: 62 x 1.0, one 2.03125, one 2^-20 ->
    #   mean = 1 + 2^-11 + 2^-26, torch rounds it to 1.0, a direct cast to 1 + 2^-10
    col = [1.0] * 62 + [2.03125, 2.0 ** -20]
    # cluster 1: two rows 2^-21 and 3 * 2^-21: rne(0.5)=0 + rne(1.5)=2 -> mean 2^-20
    #   (floor gives 2^-21, half away from zero 1.5 * 2^-20)
    rows = []
    labs = []
    for v in col:
        rows.append([v, 1.0, 0.0, 0.0])
        labs.append(0)
    rows.append([2.0 ** -21, 2.0 ** -21, 0.0, 0.0])
    labs.append(1)
    rows.append([3 * 2.0 ** -21, 2.0 ** -21, 0.0, 0.0])
    labs.append(1)
    x = np.array([rows], dtype=np.float16)
    assert float(x[0, 63, 0]) == 2.0 ** -20 and float(x[0, 64, 0]) == 2.0 ** -21
    labels = np.array([labs], dtype=np.int32)
    old = np.zeros((1, 3, D), dtype=np.float16)
    new, counts = O.det_centroid_update(x, labels, old)
    assert counts[0].tolist() == [64, 2, 0]
    assert float(new[0, 0, 0]) == 1.0                        # not 1 + 2^-10
    assert np.float16(np.float64(1 + 2.0 ** -11 + 2.0 ** -26)) != np.float16(1.0)   # direct cast differs
    assert float(new[0, 1, 0]) == 2.0 ** -20                 # (0 + 2) / 2^20 / 2
    assert float(new[0, 1, 1]) == 0.0                        # rne(0.5) twice = 0
    want = _det_update_exact(x, labels, old)
    assert np.array_equal(new.view(np.uint16), want.view(np.uint16))
