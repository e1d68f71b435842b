"""Emulation of the reference selection kernel's algorithm (test infrastructure).

TEST INFRASTRUCTURE ONLY: used by tests/ to pin ``t2t_oracle.select_rows``
(the sort-prefix statement of the selection rule) against what the
reference CUDA kernel actually computes.  It re-states, in plain Python
integer arithmetic, the per-row steps of ``k_main`` in
token2tile/operator/kernels/select_union/src/kernel.cu:

* cluster weights are packed as (size << 12) + 1 so one histogram carries
  both the key count and the cluster count (:225-239);
* a 256-bin window histogram below a predicted key ``vp`` (bins clamp at 0
  for keys >= vp and at 256 + lane beyond the window) (:162-163, 288-307);
* if the crossing bin is not strictly inside the window (s_b not in
  [1, 254]) an exact two-level radix fallback: high byte 127 - (key >> 8),
  then low byte 255 - (key & 255) of the keys in the crossing high byte
  (:314-351);
* a single cluster at the threshold selects every key >= vstar; several
  tied clusters are taken in ascending cluster order while the running tied
  size stays below ns - (size above the threshold) (:357-393, TIEFIX).

The prediction only changes how fast the kernel finds the threshold, never
the result, so the emulation accepts any predicted key.
"""
from __future__ import annotations

import numpy as np

SHF = 12
NC = 2048


def _lane_of(c):
    tid = (c % 1024) // 8
    return tid & 31


def _first_crossing(hist, start, nsP, base=0):
    """First bin b >= start (in order) where base + cumsum crosses nsP.
    Returns (b, pre, hv) or None."""
    cum = base
    for b in range(start, start + 256):
        hv = int(hist[b])
        if cum < nsP <= cum + hv:
            return b - start, cum, hv
        cum += hv
    return None


def kmain_row(keys, sizes, ns, predicted):
    """Selection of one row as the reference kernel computes it.

    keys: int16-ordered keys [2048]; sizes: int [2048]; ns: budget;
    predicted: any int key in [-32768, 32767].
    Returns (sel bool [2048], rowcnt int).
    """
    keys = np.asarray(keys, dtype=np.int64)
    sizes = np.asarray(sizes, dtype=np.int64)
    szp = (sizes << SHF) + 1
    nsP = ns << SHF
    vp = int(predicted) + 127
    hist = np.zeros(544, dtype=np.int64)
    for c in range(NC):
        tmax = 256 + _lane_of(c)
        d = min(max(vp - int(keys[c]), 0), tmax)
        hist[d] += szp[c]
    found = _first_crossing(hist, 0, nsP)
    s_b = 256 if found is None else found[0]
    if 1 <= s_b <= 254:
        vstar = vp - s_b
        packed_pre, hvb = found[1], found[2]
    else:
        hist = np.zeros(544, dtype=np.int64)
        for c in range(NC):
            hist[127 - (int(keys[c]) >> 8)] += szp[c]
        f2 = _first_crossing(hist, 0, nsP)
        bh = 127 - f2[0]
        pre = f2[1]
        for c in range(NC):
            k = int(keys[c])
            if (k >> 8) == bh:
                hist[256 + 255 - (k & 255)] += szp[c]
            else:
                hist[512 + _lane_of(c)] += szp[c]
        f3 = _first_crossing(hist, 256, nsP, base=pre)
        vstar = (bh << 8) | (255 - f3[0])
        packed_pre, hvb = f3[1], f3[2]
    sgt = packed_pre >> SHF
    if (hvb & 0xFFF) == 1:
        sel = keys >= vstar
        rowcnt = sgt + (hvb >> SHF)
        return sel, int(rowcnt)
    R = ns - sgt
    sel = keys > vstar
    rowcnt = None
    p = 0
    for c in range(NC):
        if keys[c] == vstar:
            s = int(sizes[c])
            if p < R:
                sel[c] = True
                if p + s >= R:
                    rowcnt = sgt + p + s
            p += s
    return sel, int(rowcnt)
