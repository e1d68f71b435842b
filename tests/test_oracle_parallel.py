"""The process-pool form of the oracle's full call (the CPU baseline of
bench.py) gives the output of the single-process full_call (to fp64 rounding)."""
import math

import numpy as np

from oracle import parallel as P
from oracle import t2t_oracle as O


def test_pool_full_call_equals_full_call():
    rng = np.random.default_rng(50)
    H, N, CQ, ns = 2, 4096, 24, 200
    base = rng.normal(0, 1, (H, N, 128))
    q = (base + rng.normal(0, 0.2, (H, N, 128))) / math.sqrt(128)
    k = base + rng.normal(0, 0.2, (H, N, 128))
    q, k = q.astype(np.float16), k.astype(np.float16)
    v = rng.normal(0, 1, (H, N, 128)).astype(np.float16)
    Uq, Uk = O.online_u(q.astype(np.float32), k.astype(np.float32))
    Uq, Uk = Uq.astype(np.float16), Uk.astype(np.float16)
    QU, KU = O.project(q, Uq), O.project(k, Uk)
    st = dict(Uq=Uq, Uk=Uk, ck=KU[:, np.sort(rng.choice(N, 2048, replace=False))],
              cq=QU[:, np.sort(rng.choice(N, CQ, replace=False))])
    want, _, _ = O.full_call(q, k, v, st, ns, CQ, pin_tail=32)
    got = P.full_call_pool(q, k, v, st, ns, CQ, workers=3, pin_tail=32)
    # fp64 matrix products over row subsets block differently in BLAS: equal
    # to the last bits of fp64
    assert np.allclose(got, want, rtol=0, atol=1e-14)
