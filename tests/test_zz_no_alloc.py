"""The allocation-free fused scoring + selection
(t2t_score_select_packed_noalloc) against the workspace entry point
(t2t_score_select_packed), bit for bit, on two calls in a row through the C
ABI, the second with a smaller input; both also against the oracle."""
import numpy as np
import pytest
import torch

from oracle import t2t_oracle as O

pytestmark = pytest.mark.gpu


def _case(rng, H, N, CQ):
    QU = rng.normal(0, 1, (H, N, 32)).astype(np.float16)
    ck2 = rng.normal(0, 0.5, (H, 2048, 32)).astype(np.float32)
    sizes = np.stack([rng.multinomial(N, np.ones(2048) / 2048) for _ in range(H)]).astype(np.int32)
    qlab = rng.integers(0, CQ - 1, (H, N)).astype(np.int32)     # cluster CQ-1 stays empty
    qperm, qcounts = O.stable_perm(qlab, CQ)
    return QU, ck2, sizes, qperm, qcounts


def test_noalloc_score_select_matches_workspace_entry(dev):
    from token2tile_amd import _lib, ops
    L = _lib.lib()
    rng = np.random.default_rng(2024)
    stream = torch.cuda.current_stream(dev)
    for H, N, CQ, ns in ((3, 5000, 40, 400), (2, 1500, 9, 77)):   # second call smaller
        print(f"[noalloc] H={H} N={N} CQ={CQ} ns={ns}", flush=True)
        QU, ck2, sizes, qperm, qcounts = _case(rng, H, N, CQ)
        g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        tQU, tsz, tqp, tqc = g(QU), g(sizes), g(qperm), g(qcounts)
        _, cks = ops.centroid_finalize(g(ck2))
        ns_t = torch.tensor(ns, dtype=torch.int32, device=dev)
        outs = []
        for noalloc in (False, True):
            # poison the outputs: every word must be written by the call
            unip = torch.full((H, CQ, 64), -1, dtype=torch.int32, device=dev)
            rowcnt = torch.full((H, N), -7, dtype=torch.int32, device=dev)
            if noalloc:
                rc = L.t2t_score_select_packed_noalloc(
                    tQU.data_ptr(), cks.data_ptr(), tsz.data_ptr(), tqp.data_ptr(),
                    tqc.data_ptr(), ns_t.data_ptr(), unip.data_ptr(), rowcnt.data_ptr(),
                    H, N, CQ, stream.cuda_stream)
            else:
                ws = torch.empty(ops.select_ws_bytes(H, N, CQ), dtype=torch.uint8, device=dev)
                rc = L.t2t_score_select_packed(
                    tQU.data_ptr(), cks.data_ptr(), tsz.data_ptr(), tqp.data_ptr(),
                    tqc.data_ptr(), ns_t.data_ptr(), unip.data_ptr(), rowcnt.data_ptr(),
                    H, N, CQ, ws.data_ptr(), ws.numel(), stream.cuda_stream)
            assert rc == 0, L.t2t_last_error()
            torch.cuda.synchronize(dev)
            outs.append((unip.cpu().numpy(), rowcnt.cpu().numpy()))
        assert np.array_equal(outs[0][0], outs[1][0])
        assert np.array_equal(outs[0][1], outs[1][1])
        gl = ops.score(tQU, cks).cpu().numpy()
        eu, er = O.select_union(gl, sizes, qperm, qcounts, ns)
        assert np.array_equal(outs[1][0], eu) and np.array_equal(outs[1][1], er)
