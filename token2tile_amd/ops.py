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


def _ws_for(ws, nbytes, device):
    """A caller's workspace if it is a large enough uint8 buffer on ``device``,
    else a fresh one.  Its byte count is passed to the library, which checks it."""
    if ws is not None:
        if (not isinstance(ws, torch.Tensor) or ws.dtype != torch.uint8
                or not ws.is_contiguous() or ws.device != device):
            raise ValueError(f"t2t: ws must be a contiguous uint8 tensor on {device}")
        if ws.numel() >= nbytes:
            return ws
    return _ws(nbytes, device)


_HALF = (torch.float16, torch.bfloat16)


def _check(t, shape, dtype, name, device=None):
    """The kernels take raw pointers and trust these geometries: a tensor of
    another shape, dtype or device would be read or written out of bounds."""
    dtypes = dtype if isinstance(dtype, tuple) else (dtype,)
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"t2t: {name} must be a tensor")
    if (tuple(t.shape) != tuple(shape) or t.dtype not in dtypes or not t.is_contiguous()
            or not t.is_cuda or (device is not None and t.device != device)):
        raise ValueError(f"t2t: {name} must be a contiguous {'/'.join(map(str, dtypes))} "
                         f"{tuple(shape)} tensor on {device or 'the GPU'}, got {t.dtype} "
                         f"{tuple(t.shape)} on {t.device}")


def _rows(t, H, N, D, dtype, name, device):
    """Validate an [H, N, D] view whose rows are contiguous (unit stride along
    D, 16-byte aligned) and return its (head, row) strides in elements: the
    contiguous layout, or e.g. a token-major [N, H, D] tensor seen through
    ``.transpose(0, 1)``."""
    dtypes = dtype if isinstance(dtype, tuple) else (dtype,)
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"t2t: {name} must be a tensor")
    sh, sn = (t.stride(0), t.stride(1)) if t.dim() == 3 else (0, 0)
    if (tuple(t.shape) != (H, N, D) or t.dtype not in dtypes or t.device != device
            or t.stride(2) != 1 or sh % 8 or sn % 8 or sn < D or sh < 0
            or t.data_ptr() % 16):
        raise ValueError(f"t2t: {name} must be a {'/'.join(map(str, dtypes))} [{H}, {N}, {D}] "
                         f"tensor on {device} with contiguous 16-byte aligned rows, got "
                         f"{t.dtype} {tuple(t.shape)} strides {tuple(t.stride())} on {t.device}")
    return sh, sn


def _check_ns(ns_t, device):
    if not isinstance(ns_t, torch.Tensor) or ns_t.numel() != 1 or ns_t.dtype != _i32 \
            or ns_t.device != device:
        raise ValueError(f"t2t: ns_t must be a one-element int32 tensor on {device}")


def _check_plan(plan, H, N, CQ, device):
    if (not isinstance(plan, torch.Tensor) or plan.dtype != _i32 or not plan.is_contiguous()
            or plan.device != device or plan.numel() < plan_ints(H, N, CQ)):
        raise ValueError(f"t2t: plan must be a contiguous int32 tensor of >= "
                         f"{plan_ints(H, N, CQ)} elements on {device}")


def project(x, U, out=None, stream=None):
    """fp16(x @ U): x [H, N, D] fp16/bf16, U [H, D, 32] fp16 -> [H, N, 32] fp16."""
    H, N, D = x.shape
    dev = _dev(x)
    sxh, sxn = _rows(x, H, N, D, _HALF, "x", dev)
    _check(U, (H, D, RANK), _f16, "U", dev)
    if out is None:
        out = torch.empty(H, N, RANK, dtype=_f16, device=dev)
    _check(out, (H, N, RANK), _f16, "out", dev)
    if not x.is_contiguous():
        call("t2t_project_strided", _lib.RowView(x), dtype_code(x.dtype), U, out, H, N, D, RANK,
             sxh, sxn,
             stream_handle(stream))
        return out
    call("t2t_project", x, dtype_code(x.dtype), U, out, H, N, D, RANK, stream_handle(stream))
    return out


def kmm_ws_bytes(H, N, CQ, CK=C_KEYS):
    return size_query("t2t_kmm_ws_bytes", H, N, CQ, CK)


def kmm_run(QU, KU, V, cq0, ck0, *, pin_tail=0, out=None, ws=None, stream=None,
            write_v_sorted=True):
    """One k-means maintenance call; returns a dict of the outputs.  With
    ``write_v_sorted=False`` V_sorted is neither allocated nor written (its
    entry is None): for callers that read V through kperm."""
    H, N, r = QU.shape
    CQ, CK = cq0.shape[1], ck0.shape[1]
    dev = _dev(QU)
    _check(QU, (H, N, r), _f16, "QU", dev)
    _check(KU, (H, N, r), _f16, "KU", dev)
    _check(cq0, (H, CQ, r), _f16, "cq0", dev)
    _check(ck0, (H, CK, r), _f16, "ck0", dev)
    svh, svn = _rows(V, H, N, HEAD_DIM, _HALF, "V", dev)
    o = dict(out or {})
    o.setdefault("qlab", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("cq2", torch.empty(H, CQ, r, dtype=_f16, device=dev))
    o.setdefault("klab", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("ck2", torch.empty(H, CK, r, dtype=_f32, device=dev))
    o.setdefault("qcounts", torch.empty(H, CQ, dtype=_i32, device=dev))
    o.setdefault("qperm", torch.empty(H, N, dtype=_i32, device=dev))
    o.setdefault("kcounts", torch.empty(H, CK, dtype=_i32, device=dev))
    o.setdefault("kperm", torch.empty(H, N, dtype=_i32, device=dev))
    if write_v_sorted:
        o.setdefault("V_sorted", torch.empty(H, N, HEAD_DIM, dtype=V.dtype, device=dev))
    else:
        o["V_sorted"] = None
    o.setdefault("sumv", torch.empty(H, CK, HEAD_DIM, dtype=_f16, device=dev))
    o.setdefault("lam", torch.empty(H, dtype=_f32, device=dev))
    for name, shape, dt in (("qlab", (H, N), _i32), ("cq2", (H, CQ, r), _f16),
                            ("klab", (H, N), _i32), ("ck2", (H, CK, r), _f32),
                            ("qcounts", (H, CQ), _i32), ("qperm", (H, N), _i32),
                            ("kcounts", (H, CK), _i32), ("kperm", (H, N), _i32),
                            ("V_sorted", (H, N, HEAD_DIM), V.dtype),
                            ("sumv", (H, CK, HEAD_DIM), _f16), ("lam", (H,), _f32)):
        if o[name] is not None or name != "V_sorted":
            _check(o[name], shape, dt, name, dev)
    need = kmm_ws_bytes(H, N, CQ, CK)
    ws = _ws_for(ws, need, dev)
    if V.is_contiguous():
        call("t2t_kmm_run", QU, KU, V, dtype_code(V.dtype), cq0, ck0, o["qlab"], o["cq2"],
             o["klab"], o["ck2"], o["qcounts"], o["qperm"], o["kcounts"], o["kperm"],
             o["V_sorted"], o["sumv"], o["lam"], H, N, CQ, CK, int(pin_tail), ws, ws.numel(),
             stream_handle(stream))
    else:
        call("t2t_kmm_run_strided", QU, KU, _lib.RowView(V), dtype_code(V.dtype), svh, svn, cq0,
             ck0, o["qlab"],
             o["cq2"], o["klab"], o["ck2"], o["qcounts"], o["qperm"], o["kcounts"], o["kperm"],
             o["V_sorted"], o["sumv"], o["lam"], H, N, CQ, CK, int(pin_tail), ws, ws.numel(),
             stream_handle(stream))
    return o


def vstats_ws_bytes(H, N, CK=C_KEYS):
    return size_query("t2t_vstats_ws_bytes", H, N, CK)


def vstats_gather(V, kperm, kcounts, V_sorted=None, sumv=None, lam=None, ws=None, stream=None,
                  write_v_sorted=True):
    """Reuse-call value statistics: V_sorted = V[kperm], sumv, lam.  With
    ``write_v_sorted=False`` only sumv and lam are produced (V_sorted None)."""
    H, N, D = V.shape
    CK = kcounts.shape[1]
    dev = _dev(V)
    if not write_v_sorted:
        V_sorted = None
    elif V_sorted is None:
        V_sorted = torch.empty(H, N, D, dtype=V.dtype, device=dev)
    sumv = torch.empty(H, CK, D, dtype=_f16, device=dev) if sumv is None else sumv
    lam = torch.empty(H, dtype=_f32, device=dev) if lam is None else lam
    svh, svn = _rows(V, H, N, HEAD_DIM, _HALF, "V", dev)
    _check(kperm, (H, N), _i32, "kperm", dev)
    _check(kcounts, (H, CK), _i32, "kcounts", dev)
    if V_sorted is not None:
        _check(V_sorted, (H, N, HEAD_DIM), V.dtype, "V_sorted", dev)
    _check(sumv, (H, CK, HEAD_DIM), _f16, "sumv", dev)
    _check(lam, (H,), _f32, "lam", dev)
    need = vstats_ws_bytes(H, N, CK)
    ws = _ws_for(ws, need, dev)
    if V.is_contiguous():
        call("t2t_kmm_run_vstats_gather", V, dtype_code(V.dtype), kperm, kcounts, V_sorted, sumv,
             lam, H, N, CK, ws, ws.numel(), stream_handle(stream))
    else:
        call("t2t_kmm_run_vstats_gather_strided", _lib.RowView(V), dtype_code(V.dtype), svh, svn,
             kperm, kcounts,
             V_sorted, sumv, lam, H, N, CK, ws, ws.numel(), stream_handle(stream))
    return V_sorted, sumv, lam


def vstats(V_sorted, kcounts, sumv=None, lam=None, ws=None, stream=None):
    H, N, D = V_sorted.shape
    CK = kcounts.shape[1]
    dev = _dev(V_sorted)
    sumv = torch.empty(H, CK, D, dtype=_f16, device=dev) if sumv is None else sumv
    lam = torch.empty(H, dtype=_f32, device=dev) if lam is None else lam
    _check(V_sorted, (H, N, HEAD_DIM), _HALF, "V_sorted", dev)
    _check(kcounts, (H, CK), _i32, "kcounts", dev)
    _check(sumv, (H, CK, HEAD_DIM), _f16, "sumv", dev)
    _check(lam, (H,), _f32, "lam", dev)
    need = vstats_ws_bytes(H, N, CK)
    ws = _ws_for(ws, need, dev)
    call("t2t_kmm_run_vstats", V_sorted, dtype_code(V_sorted.dtype), kcounts, sumv, lam, H, N, CK,
         ws, ws.numel(), stream_handle(stream))
    return sumv, lam


def centroid_finalize(ck2, scale=1.0 / math.sqrt(HEAD_DIM), ck16=None, cks=None, stream=None):
    """(fp16(ck2), fp16(fp32(ck2 * scale)))."""
    H, CK, r = ck2.shape
    dev = _dev(ck2)
    ck16 = torch.empty(H, CK, r, dtype=_f16, device=dev) if ck16 is None else ck16
    cks = torch.empty(H, CK, r, dtype=_f16, device=dev) if cks is None else cks
    _check(ck2, (H, CK, r), _f32, "ck2", dev)
    _check(ck16, (H, CK, r), _f16, "ck16", dev)
    _check(cks, (H, CK, r), _f16, "cks", dev)
    call("t2t_centroid_finalize", ck2, ck16, cks, float(scale), H, CK, r, stream_handle(stream))
    return ck16, cks


def score(QU, cks, out=None, stream=None):
    """gl = fp16(QU @ cks^T): [H, N, 2048] fp16."""
    H, N, r = QU.shape
    CK = cks.shape[1]
    dev = _dev(QU)
    out = torch.empty(H, N, CK, dtype=_f16, device=dev) if out is None else out
    _check(QU, (H, N, r), _f16, "QU", dev)
    _check(cks, (H, CK, r), _f16, "cks", dev)
    _check(out, (H, N, CK), _f16, "out", dev)
    call("t2t_score", QU, cks, out, H, N, CK, r, stream_handle(stream))
    return out


def select_ws_bytes(H, N, CQ):
    return size_query("t2t_select_ws_bytes", H, N, CQ)


def _check_select(dev, H, N, CQ, *, gl=None, kcounts=None, qperm=None, qcounts=None, unip=None,
                  rowcnt=None):
    if gl is not None:
        _check(gl, (H, N, C_KEYS), _f16, "gl", dev)
    _check(kcounts, (H, C_KEYS), _i32, "kcounts", dev)
    _check(qperm, (H, N), _i32, "qperm", dev)
    _check(qcounts, (H, CQ), _i32, "qcounts", dev)
    if unip is not None:
        _check(unip, (H, CQ, C_KEYS // 32), _i32, "unip", dev)
    _check(rowcnt, (H, N), _i32, "rowcnt", dev)


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
    _check_select(dev, H, N, CQ, gl=gl, kcounts=kcounts, qperm=qperm, qcounts=qcounts,
                  unip=unip, rowcnt=rowcnt)
    _check_ns(ns_t, dev)
    need = select_ws_bytes(H, N, CQ)
    ws = _ws_for(ws, need, dev)
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
    _check(QU, (H, N, RANK), _f16, "QU", dev)
    _check(cks, (H, C_KEYS, RANK), _f16, "cks", dev)
    _check_select(dev, H, N, CQ, kcounts=kcounts, qperm=qperm, qcounts=qcounts, unip=unip,
                  rowcnt=rowcnt)
    _check_ns(ns_t, dev)
    need = select_ws_bytes(H, N, CQ)
    ws = _ws_for(ws, need, dev)
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
    _check(uni, (H, CQ, CK), torch.uint8, "uni", dev)
    _check_select(dev, H, N, CQ, gl=gl, kcounts=kcounts, qperm=qperm, qcounts=qcounts,
                  rowcnt=rowcnt)
    _check_ns(ns_t, dev)
    need = select_ws_bytes(H, N, CQ)
    ws = _ws_for(ws, need, dev)
    call("t2t_select_run", gl, kcounts, qperm, qcounts, ns_t, uni, rowcnt, H, N, CQ, ws, ws.numel(),
         stream_handle(stream))
    return uni, rowcnt


def union_or_last(unip, stream=None):
    H, CQ, W = unip.shape
    _check(unip, (H, CQ, C_KEYS // 32), _i32, "unip")
    call("t2t_union_or_last", unip, H, CQ, W * 32, stream_handle(stream))
    return unip


def fast_gather(x, perm, out=None, stream=None):
    """o[h, i] = x[h, perm[h, i]] for [H, N, D] 16-bit tensors."""
    H, N, D = x.shape
    dev = _dev(x)
    out = torch.empty_like(x) if out is None else out
    _check(x, (H, N, D), _HALF, "x", dev)
    _check(perm, (H, N), _i32, "perm", dev)
    _check(out, (H, N, D), x.dtype, "out", dev)
    call("t2t_fast_gather", x, dtype_code(x.dtype), perm, out, H, N, D, stream_handle(stream))
    return out


def plan_ints(H, N, CQ):
    return size_query("t2t_tile_plan_ints", H, N, CQ)


def tile_plan(qcounts, kcounts, unip, N, plan=None, stream=None):
    H, CQ = qcounts.shape
    dev = _dev(qcounts)
    if plan is None:
        plan = torch.empty(plan_ints(H, N, CQ), dtype=_i32, device=dev)
    _check(qcounts, (H, CQ), _i32, "qcounts", dev)
    _check(kcounts, (H, C_KEYS), _i32, "kcounts", dev)
    _check(unip, (H, CQ, C_KEYS // 32), _i32, "unip", dev)
    _check_plan(plan, H, N, CQ, dev)
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


def _check_attn(dev, H, N, CQ, *, q=None, kp=None, vp=None, kcounts=None, unip=None, qperm=None,
                plan=None, out=None, lse=None, QU=None, cks=None, sumv=None, lam=None, qlab=None,
                tailw_t=None, qcounts=None, tiles=None, dt=None):
    qs = (H, N, HEAD_DIM)
    for name, t, shape, dtype in (
            ("q", q, qs, _HALF), ("kp", kp, qs, dt), ("vp", vp, qs, dt), ("out", out, qs, dt),
            ("kcounts", kcounts, (H, C_KEYS), _i32), ("qcounts", qcounts, (H, CQ), _i32),
            ("unip", unip, (H, CQ, C_KEYS // 32), _i32), ("qperm", qperm, (H, N), _i32),
            ("qlab", qlab, (H, N), _i32), ("lse", lse, (H, N), _f32),
            ("QU", QU, (H, N, RANK), _f16), ("cks", cks, (H, C_KEYS, RANK), _f16),
            ("sumv", sumv, (H, C_KEYS, HEAD_DIM), _f16), ("lam", lam, (H,), _f32),
            ("tailw_t", tailw_t, (), _f32)):
        if t is not None:
            _check(t, shape, dtype, name, dev)
    if plan is not None:
        _check_plan(plan, H, N, CQ, dev)
    if tiles is not None:
        need = size_query("t2t_centroid_tiles_bytes", H)
        if (not isinstance(tiles, torch.Tensor) or tiles.dtype != torch.uint8
                or not tiles.is_contiguous() or tiles.device != dev or tiles.numel() < need):
            raise ValueError(f"t2t: tiles must be a contiguous uint8 tensor of >= {need} bytes "
                             f"on {dev}")


def tile_attn_exact(q, kp, vp, kcounts, unip, qperm, plan, attn_out=None, lse=None, stream=None):
    """Exact attention over the unions, sorted query order."""
    H, N, D = q.shape
    CQ = unip.shape[1]
    dev = _dev(q)
    attn_out = torch.empty_like(q) if attn_out is None else attn_out
    lse = torch.empty(H, N, dtype=_f32, device=dev) if lse is None else lse
    _check_attn(dev, H, N, CQ, q=q, kp=kp, vp=vp, kcounts=kcounts, unip=unip, qperm=qperm,
                plan=plan, out=attn_out, lse=lse, dt=q.dtype)
    call("t2t_tile_attn_exact", q, kp, vp, dtype_code(q.dtype), kcounts, unip, qperm, plan,
         attn_out, lse, H, N, CQ, stream_handle(stream))
    return attn_out, lse


def tail_merge(attn_out, lse, QU, cks, sumv, kcounts, unip, qlab, qperm, lam, tailw_t, out=None,
               ws=None, stream=None):
    H, N, D = attn_out.shape
    CQ = unip.shape[1]
    dev = _dev(attn_out)
    out = torch.empty_like(attn_out) if out is None else out
    _check_attn(dev, H, N, CQ, q=attn_out, out=out, lse=lse, QU=QU, cks=cks, sumv=sumv,
                kcounts=kcounts, unip=unip, qlab=qlab, qperm=qperm, lam=lam, tailw_t=tailw_t,
                dt=attn_out.dtype)
    need = size_query("t2t_tail_merge_ws_bytes", H)
    ws = _ws_for(ws, need, dev)
    call("t2t_tail_merge", attn_out, lse, QU, cks, sumv, kcounts, unip, qlab, qperm, lam, tailw_t,
         out, dtype_code(attn_out.dtype), H, N, CQ, ws, ws.numel(), stream_handle(stream))
    return out


def centroid_tiles(cks, sumv, tiles=None, stream=None):
    """Tile image of cks / sumv staged by the residual kernel (uint8 bytes)."""
    H = cks.shape[0]
    dev = _dev(cks)
    need = size_query("t2t_centroid_tiles_bytes", H)
    tiles = _ws(need, dev) if tiles is None else tiles
    _check_attn(dev, H, 0, 0, cks=cks, sumv=sumv, tiles=tiles)
    call("t2t_centroid_tiles", cks, sumv, tiles, H, stream_handle(stream))
    return tiles


def tile_attn_exact_orig(q, kp, vp, kcounts, unip, qperm, plan, out, lse, stream=None):
    """Exact attention written at the original rows of out; lse in sorted order."""
    H, N, D = q.shape
    CQ = unip.shape[1]
    _check_attn(_dev(q), H, N, CQ, q=q, kp=kp, vp=vp, kcounts=kcounts, unip=unip, qperm=qperm,
                plan=plan, out=out, lse=lse, dt=q.dtype)
    call("t2t_tile_attn_exact_orig", q, kp, vp, dtype_code(q.dtype), kcounts, unip, qperm, plan,
         out, lse, H, N, CQ, stream_handle(stream))
    return out


def tile_attn_exact_orig_gather(q, k, kperm, vp, kcounts, unip, qperm, plan, out, lse, stream=None):
    """tile_attn_exact_orig reading K in place: k in the original order, key
    position p of the cluster order at row kperm[h, p] (no kp = k[kperm]).
    q, k and out may be strided [H, N, 128] views with contiguous rows (e.g.
    token-major tensors through ``.transpose(0, 1)``)."""
    H, N, D = q.shape
    CQ = unip.shape[1]
    dev = _dev(q)
    sq = _rows(q, H, N, HEAD_DIM, _HALF, "q", dev)
    sk = _rows(k, H, N, HEAD_DIM, q.dtype, "k", dev)
    so = _rows(out, H, N, HEAD_DIM, q.dtype, "out", dev)
    _check_attn(dev, H, N, CQ, vp=vp, kcounts=kcounts, unip=unip, qperm=qperm, plan=plan,
                lse=lse, dt=q.dtype)
    _check(kperm, (H, N), _i32, "kperm", dev)
    if q.is_contiguous() and k.is_contiguous() and out.is_contiguous():
        call("t2t_tile_attn_exact_orig_gather", q, k, kperm, vp, dtype_code(q.dtype), kcounts,
             unip, qperm, plan, out, lse, H, N, CQ, stream_handle(stream))
    else:
        call("t2t_tile_attn_exact_orig_gather_strided", _lib.RowView(q), *sq, _lib.RowView(k),
             *sk, kperm, vp, dtype_code(q.dtype), kcounts, unip, qperm, plan, _lib.RowView(out),
             *so, lse, H, N, CQ, stream_handle(stream))
    return out

def tile_attn_exact_orig_gather_kv(q, k, v, kperm, kcounts, unip, qperm, plan, out, lse,
                                   stream=None):
    """Exact attention with both gathers fused: k and v in the original order,
    key position p of the cluster order at row kperm[h, p] of each (neither
    kp nor V_sorted is stored).  q, k, v and out may be strided [H, N, 128]
    views with contiguous rows."""
    H, N, D = q.shape
    CQ = unip.shape[1]
    dev = _dev(q)
    sq = _rows(q, H, N, HEAD_DIM, _HALF, "q", dev)
    sk = _rows(k, H, N, HEAD_DIM, q.dtype, "k", dev)
    sv = _rows(v, H, N, HEAD_DIM, q.dtype, "v", dev)
    so = _rows(out, H, N, HEAD_DIM, q.dtype, "out", dev)
    _check_attn(dev, H, N, CQ, kcounts=kcounts, unip=unip, qperm=qperm, plan=plan, lse=lse,
                dt=q.dtype)
    _check(kperm, (H, N), _i32, "kperm", dev)
    call("t2t_tile_attn_exact_orig_gather_kv_strided", _lib.RowView(q), *sq, _lib.RowView(k), *sk,
         _lib.RowView(v), *sv, kperm, dtype_code(q.dtype), kcounts, unip, qperm, plan,
         _lib.RowView(out), *so, lse, H, N, CQ, stream_handle(stream))
    return out


def resid_merge_inplace(out, lse, QU, tiles, kcounts, unip, qlab, qperm, lam, tailw_t,
                        stream=None):
    """Residual + merge into the exact part held at the original rows of out
    (out may be a strided [H, N, 128] view with contiguous rows)."""
    H, N, D = out.shape
    CQ = unip.shape[1]
    dev = _dev(out)
    so = _rows(out, H, N, HEAD_DIM, _HALF, "out", dev)
    _check_attn(dev, H, N, CQ, lse=lse, QU=QU, tiles=tiles, kcounts=kcounts, unip=unip,
                qlab=qlab, qperm=qperm, lam=lam, tailw_t=tailw_t)
    if out.is_contiguous():
        call("t2t_resid_merge_inplace", out, lse, QU, tiles, kcounts, unip, qlab, qperm, lam,
             tailw_t, dtype_code(out.dtype), H, N, CQ, stream_handle(stream))
    else:
        call("t2t_resid_merge_inplace_strided", _lib.RowView(out), *so, lse, QU, tiles, kcounts,
             unip, qlab,
             qperm, lam, tailw_t, dtype_code(out.dtype), H, N, CQ, stream_handle(stream))
    return out


def attn_ws_bytes(H, N, dtype):
    return size_query("t2t_tile_attn_ws_bytes", H, N, dtype_code(dtype))


def tile_attn_run_planned(q, kp, vp, qcounts, kcounts, unip, QU, cks, sumv, lam, qlab, qperm,
                          tailw_t, out, plan, rebuild, ws=None, stream=None):
    H, N, D = q.shape
    CQ = qcounts.shape[1]
    dev = _dev(q)
    _check_attn(dev, H, N, CQ, q=q, kp=kp, vp=vp, qcounts=qcounts, kcounts=kcounts, unip=unip,
                QU=QU, cks=cks, sumv=sumv, lam=lam, qlab=qlab, qperm=qperm, tailw_t=tailw_t,
                out=out, plan=plan, dt=q.dtype)
    need = attn_ws_bytes(H, N, q.dtype)
    ws = _ws_for(ws, need, dev)
    call("t2t_tile_attn_run_planned", q, kp, vp, dtype_code(q.dtype), qcounts, kcounts, unip, QU,
         cks, sumv, lam, qlab, qperm, tailw_t, out, plan, int(bool(rebuild)), H, N, CQ, ws,
         ws.numel(), stream_handle(stream))
    return out


def fast_assign_labels(x, c, out=None, stream=None):
    H, N, D = x.shape
    C = c.shape[1]
    dev = _dev(x)
    out = torch.empty(H, N, dtype=_i32, device=dev) if out is None else out
    _check(x, (H, N, D), _f16, "x", dev)
    _check(c, (H, C, D), _f16, "c", dev)
    _check(out, (H, N), _i32, "out", dev)
    call("t2t_fast_assign", x, c, out, H, N, C, D, stream_handle(stream))
    return out


def det_centroid_update(x, labels, old, stream=None):
    """Deterministic int64 fixed-point centroid update -> (new fp16, counts)."""
    H, N, D = x.shape
    C = old.shape[1]
    dev = _dev(x)
    _check(x, (H, N, D), _f16, "x", dev)
    _check(labels, (H, N), _i32, "labels", dev)
    _check(old, (H, C, D), _f16, "old", dev)
    new = torch.empty(H, C, D, dtype=_f16, device=dev)
    counts = torch.empty(H, C, dtype=_i32, device=dev)
    ws = _ws(size_query("t2t_det_update_ws_bytes", H, N, C), dev)
    call("t2t_det_centroid_update", x, labels, old, new, counts, H, N, C, D, ws, ws.numel(),
         stream_handle(stream))
    return new, counts


def fused_update_vstats(x, labels, old, v=None, stream=None, check_labels=True):
    """fp32 centroid means (empty clusters keep ``old``), counts, and the
    fp32 per-cluster means of v when given -> (cent fp32 [H, C, D], counts
    int32 [H, C], vmean fp32 [H, C, 128] or None).  ``check_labels`` reads
    the label range back to the host (a synchronisation); callers whose
    labels come from an assignment kernel pass False."""
    H, N, D = x.shape
    C = old.shape[1]
    dev = _dev(x)
    _check(x, (H, N, D), _f16, "x", dev)
    _check(labels, (H, N), _i32, "labels", dev)
    _check(old, (H, C, D), _f16, "old", dev)
    if v is not None:
        _check(v, (H, N, HEAD_DIM), _HALF, "v", dev)
    if check_labels:
        lo, hi = (int(t) for t in torch.aminmax(labels))
        if lo < 0 or hi >= C:
            raise ValueError(f"t2t: labels must lie in [0, {C}), got [{lo}, {hi}]")
    cent = torch.empty(H, C, D, dtype=_f32, device=dev)
    counts = torch.empty(H, C, dtype=_i32, device=dev)
    vmean = None if v is None else torch.empty(H, C, HEAD_DIM, dtype=_f32, device=dev)
    ws = _ws(size_query("t2t_det_update_ws_bytes", H, N, C), dev)
    call("t2t_fused_update_vstats", x, labels, old, v, dtype_code(v.dtype) if v is not None else 0,
         cent, counts, vmean, H, N, C, D, ws, ws.numel(), stream_handle(stream))
    return cent, counts, vmean


def gram(x, stream=None):
    """x^T x / N per head in fp64: [H, D, D]."""
    H, N, D = x.shape
    _check(x, (H, N, D), _HALF, "x", _dev(x))
    G = torch.empty(H, D, D, dtype=torch.float64, device=_dev(x))
    nws = size_query("t2t_gram_ws_bytes", H, N, D)
    ws = torch.empty(nws, dtype=torch.uint8, device=_dev(x))
    call("t2t_gram", x, dtype_code(x.dtype), G, H, N, D, ws, nws, stream_handle(stream))
    return G
