"""Drop-in replacements for the reference operator's three extension loaders.

``token2tile/operator/deploy_step.py:59-101`` builds three torch extensions
(``load_select_union_ext``, ``load_tile_attn_ext``, ``load_kmm_ext``) and calls
their methods from ``MaskedStepDeploy.step``.  The loaders below return objects
with the same method names and positional arguments, backed by the C ABI of
``libt2t_hip.so``, so the reference's operator file can run on MI355X by
swapping its three loaders for these.

Differences a caller can observe:

* the reference's private scratch buffers (``_selector_partial``,
  ``_selector_off``, ``_tsv``, ``_qoff_v``, ``vbase32``, ``nsplit32``) are
  accepted and ignored; the HIP kernels use a workspace cached here per
  (device, shape), allocated on first use;
* a ``plan`` buffer smaller than this library's plan (``t2t_tile_plan_ints``)
  is paired with a private plan of the right size, keyed by the caller
  buffer's address, so snapshot reuse (``rebuild=False``) still finds the plan
  built on the rebuild call;
* q/k/v may be fp16 or bf16 (the reference accepts fp16 only).
"""
from __future__ import annotations

import torch

from . import ops


class _WsCache:
    def __init__(self):
        self._bufs = {}

    def get(self, key, nbytes, device):
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


class KmmExt:
    """``kmeans_maintain`` extension (kernels/kmeans_maintain/main.cpp)."""

    def __init__(self):
        self._ws = _WsCache()

    def run(self, QU, KU, v, cq, ck, qlab, cq2, klab, ck2, qcounts, qperm, kcounts, kperm,
            vp, sumv, lam, pin_tail):
        H, N, _ = QU.shape
        CQ, CK = cq.shape[1], ck.shape[1]
        ws = self._ws.get(("kmm", QU.device, H, N, CQ, CK), ops.kmm_ws_bytes(H, N, CQ, CK),
                          QU.device)
        ops.kmm_run(QU, KU, v, cq, ck, pin_tail=int(pin_tail), ws=ws,
                    out={"qlab": qlab, "cq2": cq2, "klab": klab, "ck2": ck2, "qcounts": qcounts,
                         "qperm": qperm, "kcounts": kcounts, "kperm": kperm, "V_sorted": vp,
                         "sumv": sumv, "lam": lam})

    def run_vstats(self, vp, counts, sumv, lam):
        H, N, _ = vp.shape
        CK = counts.shape[1]
        ws = self._ws.get(("vst", vp.device, H, N, CK), ops.vstats_ws_bytes(H, N, CK), vp.device)
        ops.vstats(vp, counts, sumv, lam, ws=ws)

    def run_vstats_gather(self, v, kperm, counts, vp, sumv, lam):
        H, N, _ = v.shape
        CK = counts.shape[1]
        ws = self._ws.get(("vst", v.device, H, N, CK), ops.vstats_ws_bytes(H, N, CK), v.device)
        ops.vstats_gather(v, kperm, counts, vp, sumv, lam, ws=ws)


class SelectUnionExt:
    """``select_union`` extension (kernels/select_union/src/main.cpp)."""

    def __init__(self):
        self._ws = _WsCache()

    def _wsbuf(self, gl, CQ):
        H, N, _ = gl.shape
        return self._ws.get((gl.device, H, N, CQ), ops.select_ws_bytes(H, N, CQ), gl.device)

    def run(self, gl, counts, qperm, tile_sizes, ns_t, uni, rowcnt):
        ops.select_union_bytes(gl, counts, qperm, tile_sizes, ns_t, uni=uni, rowcnt=rowcnt,
                               ws=self._wsbuf(gl, tile_sizes.shape[1]))

    def run_split(self, gl, counts, qperm, tile_sizes, split_cap, ns_t, uni, rowcnt,
                  virtual_sizes, off, vbase, nsplit):
        # the union does not depend on how rows are split across work-groups
        if int(split_cap) < 1:
            raise ValueError("t2t: split_cap must be >= 1")
        self.run(gl, counts, qperm, tile_sizes, ns_t, uni, rowcnt)

    def run_packed(self, gl, counts, qperm, tile_sizes, ns_t, partial, unip, rowcnt, off):
        ops.select_union(gl, counts, qperm, tile_sizes, ns_t, unip=unip, rowcnt=rowcnt,
                         ws=self._wsbuf(gl, tile_sizes.shape[1]))

    def run_split_packed(self, gl, counts, qperm, tile_sizes, split_cap, ns_t, partial, unip,
                         rowcnt, tsv, qoff_v, vbase32, nsplit32):
        ops.select_union(gl, counts, qperm, tile_sizes, ns_t, unip=unip, rowcnt=rowcnt,
                         ws=self._wsbuf(gl, tile_sizes.shape[1]), split_cap=int(split_cap))


class TileAttnExt:
    """``tile_attn`` extension (kernels/tile_attn/main.cpp)."""

    def __init__(self):
        self._plans = {}
        self._ws = _WsCache()

    def _plan_for(self, plan, H, N, CQ):
        need = ops.plan_ints(H, N, CQ)
        if plan is not None and plan.numel() >= need:
            return plan
        key = (None if plan is None else plan.data_ptr(), H, N, CQ)
        own = self._plans.get(key)
        if own is None:
            dev = plan.device if plan is not None else torch.device("cuda")
            own = torch.empty(need, dtype=torch.int32, device=dev)
            self._plans[key] = own
        return own

    @staticmethod
    def _packed(union_bits):
        H, CQ, nbytes = union_bits.shape
        return union_bits.contiguous().view(torch.int32).reshape(H, CQ, nbytes // 4)

    def run_planned(self, q, kp, vp, tile_sizes, counts, union_bits, QU, cks, sumv, lam, qlab,
                    qperm, tailw_t, out, plan, rebuild):
        H, N, _ = q.shape
        CQ = tile_sizes.shape[1]
        ws = self._ws.get((q.device, H, N), ops.attn_ws_bytes(H, N, q.dtype), q.device)
        ops.tile_attn_run_planned(q, kp, vp, tile_sizes, counts, self._packed(union_bits), QU, cks,
                                  sumv, lam, qlab, qperm, tailw_t, out,
                                  self._plan_for(plan, H, N, CQ), bool(rebuild), ws=ws)
        return out

    def run(self, q, kp, vp, tile_sizes, counts, union_bits, QU, cks, sumv, lam, qlab, qperm,
            tailw_t, out):
        return self.run_planned(q, kp, vp, tile_sizes, counts, union_bits, QU, cks, sumv, lam,
                                qlab, qperm, tailw_t, out, None, True)


def load_kmm_ext(verbose=False):
    """Replaces deploy_step.py:84-101."""
    ops._lib.lib()
    return KmmExt()


def load_select_union_ext(verbose=False):
    """Replaces deploy_step.py:59-67."""
    ops._lib.lib()
    return SelectUnionExt()


def load_tile_attn_ext(verbose=False):
    """Replaces deploy_step.py:70-81."""
    ops._lib.lib()
    return TileAttnExt()
