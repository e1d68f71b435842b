"""Tensor-level wrappers of the HIP entry points (one per stage).

Each wrapper validates shapes on the host, allocates outputs that are not
passed in, and enqueues the HIP kernels on ``stream`` (default: torch's
current stream).  There is no CPU path: every function requires the HIP
library and CUDA (ROCm) tensors.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import call, dtype_code, size_query, stream_handle

C_KEYS = 2048
HEAD_DIM = 128
RANK = 32

_i32, _f16, _f32 = torch.int32, torch.float16, torch.float32


def _dev(t):
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        raise ValueError("t2t: expected a GPU tensor")
    return t.device


def _ws(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _check(t, shape, dtype, name):
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"t2t: {name} must be contiguous {dtype} {tuple(shape)}, "
                         f"got {t.dtype} {tuple(t.shape)}")


def project(x, U, out=None, stream=None):
    """fp16(x @ U): x [H, N, D] fp16/bf16, U [H, D, 32] fp16 -> [H, N, 32] fp16."""
    H, N, D = x.shape
    _check(U, (H, D, RANK), _f16, "U")
    if out is None:
        out = torch.empty(H, N, RANK, dtype=_f16, device=_dev(x))
    call("t2t_project", x, dtype_code(x.dtype), U, out, H, N, D, RANK, stream_handle(stream))
    return out


def kmm_ws_bytes(H, N, CQ, CK=C_KEYS):
    return size_query("t2t_kmm_ws_bytes", H, N, CQ, CK)


def kmm_run(QU, KU, V, cq0, ck0, *, pin_tail=0, out=None, ws=None, stream=None):
    """One k-means maintenance call; returns a dict of the outputs."""
    H, N, r = QU.shape
    CQ, CK = cq0.shape[1], ck0.shape[1]
    dev = _dev(QU)
    _check(KU, (H, N, r), _f16, "KU")
    _check(cq0, (H, CQ, r), _f16, "cq0")
    _check(ck0, (H, CK, r), _f16, "ck0")
    if V.shape != (H, N, HEAD_DIM):
        raise ValueError("t2t: V must be [H, N, 128]")
    o = dict(out or {})
    o.setdefault("qlab", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("cq2", torch.empty(H, CQ, r, dtype=_f16, device=dev))
    o.setdefault("klab", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("ck2", torch.empty(H, CK, r, dtype=_f32, device=dev))
    o.setdefault("qcounts", torch.empty(H, CQ, dtype=_i32, device=dev))
    o.setdefault("qperm", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("kcounts", torch.empty(H, CK, dtype=_i32, device=dev))
    o.setdefault("kperm", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("V_sorted", torch.empty_like(V))
    o.setdefault("sumv", torch.empty(H, CK, HEAD_DIM, dtype=_f16, device=dev))
    o.setdefault("lam", torch.empty(H, dtype=_f32, device=dev))
    need = kmm_ws_bytes(H, N, CQ, CK)
    if ws is None or ws.numel() < need:
        ws = _ws(need, dev)
    call("t2t_kmm_run", QU, KU, V, dtype_code(V.dtype), cq0, ck0, o["qlab"], o["cq2"], o["klab"],
         o["ck2"], o["qcounts"], o["qperm"], o["kcounts"], o["kperm"], o["V_sorted"], o["sumv"],
         o["lam"], H, N, CQ, CK, int(pin_tail), ws, ws.numel(), stream_handle(stream))
    return o


def vstats_ws_bytes(H, N, CK=C_KEYS):
    return size_query("t2t_vstats_ws_bytes", H, N, CK)


def vstats_gather(V, kperm, kcounts, V_sorted=None, sumv=None, lam=None, ws=None, stream=None):
    """Reuse-call value statistics: V_sorted = V[kperm], sumv, lam."""
    H, N, D = V.shape
    CK = kcounts.shape[1]
    dev = _dev(V)
    V_sorted = torch.empty_like(V) if V_sorted is None else V_sorted
    sumv = torch.empty(H, CK, D, dtype=_f16, device=dev) if sumv is None else sumv
    lam = torch.empty(H, dtype=_f32, device=dev) if lam is None else lam
    need = vstats_ws_bytes(H, N, CK)
    if ws is None or ws.numel() < need:
        ws = _ws(need, dev)
    call("t2t_kmm_run_vstats_gather", V, dtype_code(V.dtype), kperm, kcounts, V_sorted, sumv, lam,
         H, N, CK, ws, ws.numel(), stream_handle(stream))
    return V_sorted, sumv, lam


def vstats(V_sorted, kcounts, sumv=None, lam=None, ws=None, stream=None):
    H, N, D = V_sorted.shape
    CK = kcounts.shape[1]
    dev = _dev(V_sorted)
    sumv = torch.empty(H, CK, D, dtype=_f16, device=dev) if sumv is None else sumv
    lam = torch.empty(H, dtype=_f32, device=dev) if lam is None else lam
    need = vstats_ws_bytes(H, N, CK)
    if ws is None or ws.numel() < need:
        ws = _ws(need, dev)
    call("t2t_kmm_run_vstats", V_sorted, dtype_code(V_sorted.dtype), kcounts, sumv, lam, H, N, CK,
         ws, ws.numel(), stream_handle(stream))
    return sumv, lam


def centroid_finalize(ck2, scale=1.0 / math.sqrt(HEAD_DIM), ck16=None, cks=None, stream=None):
    """(fp16(ck2), fp16(fp32(ck2 * scale)))."""
    H, CK, r = ck2.shape
    dev = _dev(ck2)
    ck16 = torch.empty(H, CK, r, dtype=_f16, device=dev) if ck16 is None else ck16
    cks = torch.empty(H, CK, r, dtype=_f16, device=dev) if cks is None else cks
    call("t2t_centroid_finalize", ck2, ck16, cks, float(scale), H, CK, r, stream_handle(stream))
    return ck16, cks


def score(QU, cks, out=None, stream=None):
    """gl = fp16(QU @ cks^T): [H, N, 2048] fp16."""
    H, N, r = QU.shape
    CK = cks.shape[1]
    out = torch.empty(H, N, CK, dtype=_f16, device=_dev(QU)) if out is None else out
    call("t2t_score", QU, cks, out, H, N, CK, r, stream_handle(stream))
    return out


def select_ws_bytes(H, N, CQ):
    return size_query("t2t_select_ws_bytes", H, N, CQ)


def select_union(gl, kcounts, qperm, qcounts, ns_t, unip=None, rowcnt=None, ws=None,
                 split_cap=0, stream=None):
    """Packed union [H, CQ, 64] int32 and rowcnt [H, N] int32."""
    H, N, CK = gl.shape
    CQ = qcounts.shape[1]
    dev = _dev(gl)
    if CK != C_KEYS:
        raise ValueError("t2t: selection requires 2048 key clusters")
    unip = torch.empty(H, CQ, CK // 32, dtype=_i32, device=dev) if unip is None else unip
    rowcnt = torch.empty(H, N, dtype=_i32, device=dev) if rowcnt is None else rowcnt
    need = select_ws_bytes(H, N, CQ)
    if ws is None or ws.numel() < need:
        ws = _ws(need, dev)
    if split_cap:
        call("t2t_select_run_split_packed", gl, kcounts, qperm, qcounts, int(split_cap), ns_t, unip,
             rowcnt, H, N, CQ, ws, ws.numel(), stream_handle(stream))
    else:
        call("t2t_select_run_packed", gl, kcounts, qperm, qcounts, ns_t, unip, rowcnt, H, N, CQ, ws,
             ws.numel(), stream_handle(stream))
    return unip, rowcnt


def score_select(QU, cks, kcounts, qperm, qcounts, ns_t, unip=None, rowcnt=None, ws=None,
                 stream=None):
    """Fused scoring + selection: packed union [H, CQ, 64] int32 and rowcnt
    [H, N], identical to score() followed by select_union()."""
    H, N, r = QU.shape
    CQ = qcounts.shape[1]
    dev = _dev(QU)
    if cks.shape != (H, C_KEYS, RANK):
        raise ValueError("t2t: score_select requires cks [H, 2048, 32]")
    unip = torch.empty(H, CQ, C_KEYS // 32, dtype=_i32, device=dev) if unip is None else unip
    rowcnt = torch.empty(H, N, dtype=_i32, device=dev) if rowcnt is None else rowcnt
    need = select_ws_bytes(H, N, CQ)
    if ws is None or ws.numel() < need:
        ws = _ws(need, dev)
    call("t2t_score_select_packed", QU, cks, kcounts, qperm, qcounts, ns_t, unip, rowcnt, H, N, CQ,
         ws, ws.numel(), stream_handle(stream))
    return unip, rowcnt


def select_union_bytes(gl, kcounts, qperm, qcounts, ns_t, uni=None, rowcnt=None, ws=None,
                       stream=None):
    """Byte-per-cluster union [H, CQ, 2048] uint8 (the reference's `run`)."""
    H, N, CK = gl.shape
    CQ = qcounts.shape[1]
    dev = _dev(gl)
    uni = torch.empty(H, CQ, CK, dtype=torch.uint8, device=dev) if uni is None else uni
    rowcnt = torch.empty(H, N, dtype=_i32, device=dev) if rowcnt is None else rowcnt
    _check(uni, (H, CQ, CK), torch.uint8, "uni")
    _check(rowcnt, (H, N), _i32, "rowcnt")
    need = select_ws_bytes(H, N, CQ)
    if ws is None or ws.numel() < need:
        ws = _ws(need, dev)
    call("t2t_select_run", gl, kcounts, qperm, qcounts, ns_t, uni, rowcnt, H, N, CQ, ws, ws.numel(),
         stream_handle(stream))
    return uni, rowcnt


def union_or_last(unip, stream=None):
    H, CQ, W = unip.shape
    call("t2t_union_or_last", unip, H, CQ, W * 32, stream_handle(stream))
    return unip


def fast_gather(x, perm, out=None, stream=None):
    """o[h, i] = x[h, perm[h, i]] for [H, N, D] 16-bit tensors."""
    H, N, D = x.shape
    out = torch.empty_like(x) if out is None else out
    call("t2t_fast_gather", x, dtype_code(x.dtype), perm, out, H, N, D, stream_handle(stream))
    return out


def plan_ints(H, N, CQ):
    return size_query("t2t_tile_plan_ints", H, N, CQ)


def tile_plan(qcounts, kcounts, unip, N, plan=None, stream=None):
    H, CQ = qcounts.shape
    if plan is None:
        plan = torch.empty(plan_ints(H, N, CQ), dtype=_i32, device=_dev(qcounts))
    call("t2t_tile_plan", qcounts, kcounts, unip, plan, H, N, CQ, stream_handle(stream))
    return plan


def plan_views(plan, H, N, CQ):
    """Named views of a plan buffer (k_off, kvlen, ntask, tasks)."""
    maxT = CQ + (N + 127) // 128 + 1  # tasks of <= 128 queries
    o = 0
    k_off = plan[o:o + H * 2049].view(H, 2049); o += H * 2049
    kvlen = plan[o:o + H * CQ].view(H, CQ); o += H * CQ
    ntask = plan[o:o + H]; o += H
    tasks = plan[o:o + H * maxT * 4].view(H, maxT, 4)
    return dict(k_off=k_off, kvlen=kvlen, ntask=ntask, tasks=tasks)


def tile_attn_exact(q, kp, vp, kcounts, unip, qperm, plan, attn_out=None, lse=None, stream=None):
    """Exact attention over the unions, sorted query order."""
    H, N, D = q.shape
    CQ = unip.shape[1]
    dev = _dev(q)
    attn_out = torch.empty_like(q) if attn_out is None else attn_out
    lse = torch.empty(H, N, dtype=_f32, device=dev) if lse is None else lse
    call("t2t_tile_attn_exact", q, kp, vp, dtype_code(q.dtype), kcounts, unip, qperm, plan,
         attn_out, lse, H, N, CQ, stream_handle(stream))
    return attn_out, lse


def tail_merge(attn_out, lse, QU, cks, sumv, kcounts, unip, qlab, qperm, lam, tailw_t, out=None,
               ws=None, stream=None):
    H, N, D = attn_out.shape
    CQ = unip.shape[1]
    out = torch.empty_like(attn_out) if out is None else out
    need = size_query("t2t_tail_merge_ws_bytes", H)
    if ws is None or ws.numel() < need:
        ws = _ws(need, _dev(attn_out))
    call("t2t_tail_merge", attn_out, lse, QU, cks, sumv, kcounts, unip, qlab, qperm, lam, tailw_t,
         out, dtype_code(attn_out.dtype), H, N, CQ, ws, ws.numel(), stream_handle(stream))
    return out


def centroid_tiles(cks, sumv, tiles=None, stream=None):
    """Tile image of cks / sumv staged by the residual kernel (uint8 bytes)."""
    H = cks.shape[0]
    need = size_query("t2t_centroid_tiles_bytes", H)
    tiles = _ws(need, _dev(cks)) if tiles is None else tiles
    call("t2t_centroid_tiles", cks, sumv, tiles, H, stream_handle(stream))
    return tiles


def tile_attn_exact_orig(q, kp, vp, kcounts, unip, qperm, plan, out, lse, stream=None):
    """Exact attention written at the original rows of out; lse in sorted order."""
    H, N, D = q.shape
    CQ = unip.shape[1]
    call("t2t_tile_attn_exact_orig", q, kp, vp, dtype_code(q.dtype), kcounts, unip, qperm, plan,
         out, lse, H, N, CQ, stream_handle(stream))
    return out


def resid_merge_inplace(out, lse, QU, tiles, kcounts, unip, qlab, qperm, lam, tailw_t,
                        stream=None):
    """Residual + merge into the exact part held at the original rows of out."""
    H, N, D = out.shape
    CQ = unip.shape[1]
    call("t2t_resid_merge_inplace", out, lse, QU, tiles, kcounts, unip, qlab, qperm, lam, tailw_t,
         dtype_code(out.dtype), H, N, CQ, stream_handle(stream))
    return out


def attn_ws_bytes(H, N, dtype):
    return size_query("t2t_tile_attn_ws_bytes", H, N, dtype_code(dtype))


def tile_attn_run_planned(q, kp, vp, qcounts, kcounts, unip, QU, cks, sumv, lam, qlab, qperm,
                          tailw_t, out, plan, rebuild, ws=None, stream=None):
    H, N, D = q.shape
    CQ = qcounts.shape[1]
    need = attn_ws_bytes(H, N, q.dtype)
    if ws is None or ws.numel() < need:
        ws = _ws(need, _dev(q))
    call("t2t_tile_attn_run_planned", q, kp, vp, dtype_code(q.dtype), qcounts, kcounts, unip, QU,
         cks, sumv, lam, qlab, qperm, tailw_t, out, plan, int(bool(rebuild)), H, N, CQ, ws,
         ws.numel(), stream_handle(stream))
    return out


def fast_assign_labels(x, c, out=None, stream=None):
    H, N, D = x.shape
    C = c.shape[1]
    out = torch.empty(H, N, dtype=_i32, device=_dev(x)) if out is None else out
    call("t2t_fast_assign", x, c, out, H, N, C, D, stream_handle(stream))
    return out


def det_centroid_update(x, labels, old, stream=None):
    """Deterministic int64 fixed-point centroid update -> (new fp16, counts)."""
    H, N, D = x.shape
    C = old.shape[1]
    dev = _dev(x)
    new = torch.empty(H, C, D, dtype=_f16, device=dev)
    counts = torch.empty(H, C, dtype=_i32, device=dev)
    ws = _ws(size_query("t2t_det_update_ws_bytes", H, N, C), dev)
    call("t2t_det_centroid_update", x, labels, old, new, counts, H, N, C, D, ws, ws.numel(),
         stream_handle(stream))
    return new, counts


def gram(x, stream=None):
    """x^T x / N per head in fp64: [H, D, D]."""
    H, N, D = x.shape
    G = torch.empty(H, D, D, dtype=torch.float64, device=_dev(x))
    call("t2t_gram", x, dtype_code(x.dtype), G, H, N, D, stream_handle(stream))
    return G
