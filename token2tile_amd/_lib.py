"""ctypes binding of libt2t_hip.so (the C ABI declared in include/t2t_hip.h).

The library is built in-tree by ``python -m token2tile_amd.build``; loading
never builds and never falls back: a missing library raises.  torch is
imported first so that the library binds to the HIP runtime torch already
loaded (same soname), which makes torch's device pointers and streams valid
arguments.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_longlong, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libt2t_hip.so"

F16, BF16 = 0, 1
_P = c_void_p

# name -> (restype, argtypes)
SIGNATURES = {
    "t2t_last_error": (ctypes.c_char_p, []),
    "t2t_abi_version": (c_int, []),
    "t2t_project": (c_int, [_P, c_int, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "t2t_kmm_ws_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "t2t_kmm_run": (c_int, [_P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                            c_int, c_int, c_int, c_int, c_int, _P, c_size_t, _P]),
    "t2t_vstats_ws_bytes": (c_size_t, [c_int, c_int, c_int]),
    "t2t_kmm_run_vstats_gather": (c_int, [_P, c_int, _P, _P, _P, _P, _P, c_int, c_int, c_int,
                                          _P, c_size_t, _P]),
    "t2t_kmm_run_vstats": (c_int, [_P, c_int, _P, _P, _P, c_int, c_int, c_int, _P, c_size_t, _P]),
    "t2t_centroid_finalize": (c_int, [_P, _P, _P, c_float, c_int, c_int, c_int, _P]),
    "t2t_score": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "t2t_select_ws_bytes": (c_size_t, [c_int, c_int, c_int]),
    "t2t_score_select_packed": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P,
                                        c_size_t, _P]),
    "t2t_score_select_noalloc_max_ints": (c_size_t, []),
    "t2t_score_select_packed_noalloc": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int,
                                                c_int, _P]),
    "t2t_select_run_packed": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P,
                                      c_size_t, _P]),
    "t2t_select_run_split_packed": (c_int, [_P, _P, _P, _P, c_int, _P, _P, _P, c_int, c_int,
                                            c_int, _P, c_size_t, _P]),
    "t2t_select_run": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P, c_size_t, _P]),
    "t2t_union_or_last": (c_int, [_P, c_int, c_int, c_int, _P]),
    "t2t_fast_gather": (c_int, [_P, c_int, _P, _P, c_int, c_int, c_int, _P]),
    "t2t_tile_plan_ints": (c_size_t, [c_int, c_int, c_int]),
    "t2t_tile_plan": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P]),
    "t2t_tile_attn_exact": (c_int, [_P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int,
                                    c_int, _P]),
    "t2t_centroid_tiles_bytes": (c_size_t, [c_int]),
    "t2t_centroid_tiles": (c_int, [_P, _P, _P, c_int, _P]),
    "t2t_tile_attn_exact_orig": (c_int, [_P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int,
                                         c_int, _P]),
    "t2t_tile_attn_exact_orig_gather": (c_int, [_P, _P, _P, _P, c_int, _P, _P, _P, _P, _P, _P,
                                                c_int, c_int, c_int, _P]),
    "t2t_tile_attn_exact_orig_gather_kv_strided": (c_int, [_P, c_longlong, c_longlong, _P, c_longlong,
                                                           c_longlong, _P, c_longlong, c_longlong,
                                                           _P, c_int, _P, _P, _P, _P, _P,
                                                           c_longlong, c_longlong, _P, c_int,
                                                           c_int, c_int, _P]),
    "t2t_project_strided": (c_int, [_P, c_int, _P, _P, c_int, c_int, c_int, c_int, c_longlong,
                                    c_longlong, _P]),
    "t2t_kmm_run_strided": (c_int, [_P, _P, _P, c_int, c_longlong, c_longlong] + [_P] * 13 +
                            [c_int] * 5 + [_P, c_size_t, _P]),
    "t2t_kmm_run_vstats_gather_strided": (c_int, [_P, c_int, c_longlong, c_longlong, _P, _P, _P,
                                                  _P, _P, c_int, c_int, c_int, _P, c_size_t, _P]),
    "t2t_tile_attn_exact_orig_gather_strided": (c_int, [_P, c_longlong, c_longlong, _P, c_longlong,
                                                        c_longlong, _P, _P, c_int, _P, _P, _P, _P,
                                                        _P, c_longlong, c_longlong, _P, c_int,
                                                        c_int, c_int, _P]),
    "t2t_resid_merge_inplace_strided": (c_int, [_P, c_longlong, c_longlong] + [_P] * 9 +
                                        [c_int] * 4 + [_P]),
    "t2t_resid_merge_inplace": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int,
                                        c_int, c_int, _P]),
    "t2t_tail_merge_ws_bytes": (c_size_t, [c_int]),
    "t2t_tail_merge": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int,
                               c_int, c_int, _P, c_size_t, _P]),
    "t2t_tile_attn_ws_bytes": (c_size_t, [c_int, c_int, c_int]),
    "t2t_tile_attn_run_planned": (c_int, [_P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                          _P, _P, _P, c_int, c_int, c_int, c_int, _P, c_size_t,
                                          _P]),
    "t2t_fast_assign": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "t2t_det_update_ws_bytes": (c_size_t, [c_int, c_int, c_int]),
    "t2t_det_centroid_update": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P,
                                        c_size_t, _P]),
    "t2t_fused_update_vstats": (c_int, [_P, _P, _P, _P, c_int, _P, _P, _P, c_int, c_int, c_int,
                                        c_int, _P, c_size_t, _P]),
    "t2t_gram_ws_bytes": (c_size_t, [c_int, c_int, c_int]),
    "t2t_gram": (c_int, [_P, c_int, _P, c_int, c_int, c_int, _P, c_size_t, _P]),
}

_lib = None


def lib():
    """The loaded library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m token2tile_amd.build` "
                "(the HIP kernels have no fallback)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class RowView:
    """A strided tensor whose geometry the caller has validated and whose
    strides it passes to a ``*_strided`` entry point beside the pointer."""
    __slots__ = ("t",)

    def __init__(self, t):
        self.t = t


def ptr(t):
    """Device pointer of a tensor (None -> NULL).  Plain tensors must be
    contiguous; a RowView passes its (validated) strided tensor's pointer."""
    if t is None:
        return None
    if isinstance(t, RowView):
        return t.t.data_ptr()
    if not isinstance(t, torch.Tensor):
        return t
    if not t.is_contiguous():
        raise ValueError("t2t: tensors passed to the HIP library must be contiguous")
    return t.data_ptr()


def dtype_code(dt):
    if dt == torch.float16:
        return F16
    if dt == torch.bfloat16:
        return BF16
    raise TypeError(f"t2t: unsupported dtype {dt} (fp16 or bf16)")


def stream_handle(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def call(name, *args):
    """Call a status-returning entry point; raise RuntimeError on failure."""
    fn = getattr(lib(), name)
    rc = fn(*[ptr(a) if isinstance(a, (torch.Tensor, RowView)) else a for a in args])
    if rc != 0:
        msg = lib().t2t_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def size_query(name, *args):
    return int(getattr(lib(), name)(*args))
