"""The C-ABI library loads, exports every symbol include/t2t_hip.h declares,
and rejects bad arguments with an error code and a message (no GPU needed:
argument validation happens before any HIP call)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "t2t_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t2t_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from token2tile_amd import _lib
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} missing from the ctypes signature table"
    assert set(_lib.SIGNATURES) == set(names)
    assert L.t2t_abi_version() == 101


def test_workspace_queries():
    from token2tile_amd import ops
    assert ops.kmm_ws_bytes(40, 75600, 512) > 40 * 75600 * 4
    assert ops.select_ws_bytes(40, 75600, 512) >= 40 * 513 * 4
    assert ops.plan_ints(40, 75600, 512) > 40 * 2049
    assert ops.vstats_ws_bytes(2, 16384) >= 2 * 2048 * 128 * 4


@pytest.mark.parametrize("call", [
    lambda L: L.t2t_project(None, 0, None, None, 1, 1, 128, 32, None),
    lambda L: L.t2t_score(None, None, None, 1, 1, 2048, 32, None),
    lambda L: L.t2t_fast_gather(None, 0, None, None, 1, 1, 128, None),
    lambda L: L.t2t_tile_plan(None, None, None, None, 1, 1, 1, None),
])
def test_null_pointers_rejected(call):
    from token2tile_amd import _lib
    L = _lib.lib()
    assert call(L) == 1
    assert b"null" in L.t2t_last_error()


def test_bad_sizes_rejected():
    from token2tile_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    assert L.t2t_project(p, 0, p, p, 1, 1, 128, 16, None) == 1         # r != 32
    assert L.t2t_project(p, 7, p, p, 1, 1, 128, 32, None) == 1         # dtype
    assert L.t2t_select_run_packed(p, p, p, p, p, p, p, 1, 524288, 4, p, 1 << 20, None) == 1
    assert L.t2t_kmm_run(p, p, p, 0, p, p, p, p, p, p, p, p, p, p, p, p, p,
                         1, 100, 8, 2048, 101, p, 1 << 30, None) == 1    # pin_tail > N
    assert L.t2t_kmm_run(p, p, p, 0, p, p, p, p, p, p, p, p, p, p, p, p, p,
                         1, 100, 8, 2048, 0, p, 16, None) == 2           # workspace too small
    assert b"workspace" in L.t2t_last_error()
    assert L.t2t_select_run_split_packed(p, p, p, p, 0, p, p, p, 1, 8, 4, p, 1 << 20, None) == 1


def test_noalloc_select_rejects_oversized_scratch():
    """The allocation-free fused selection refuses shapes whose offsets do not
    fit its static scratch, before touching the GPU."""
    from token2tile_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    cap = L.t2t_score_select_noalloc_max_ints()
    assert cap == 64 * 4097
    assert L.t2t_score_select_packed_noalloc(p, p, p, p, p, p, p, p, 65, 8192, 4096, None) == 4
    assert b"static scratch" in L.t2t_last_error()
    assert L.t2t_score_select_packed_noalloc(None, p, p, p, p, p, p, p, 1, 8192, 16, None) == 1


def test_attention_entry_points_reject_bad_arguments():
    """The exact-attention and residual entries reject a bad dtype, sizes
    outside their limits, strides the kernels cannot address and a short
    workspace, each with its error code, before any launch."""
    from token2tile_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    exact = lambda dtype, H, N, CQ: L.t2t_tile_attn_exact(p, p, p, dtype, p, p, p, p, p, p, H, N,
                                                          CQ, None)
    assert exact(7, 1, 64, 4) == 1 and b"dtype" in L.t2t_last_error()
    assert exact(1, 0, 64, 4) == 1
    assert exact(1, 1, 1 << 24, 4) == 1                   # row indices are 24-bit in LDS
    assert L.t2t_tail_merge(p, p, p, p, p, p, p, p, p, p, p, p, 1, 2, 64, 4, p, 16, None) == 2
    assert b"workspace" in L.t2t_last_error()

    def strided(q_rs=128, k_rs=128, N=64, o_rs=128):
        return L.t2t_tile_attn_exact_orig_gather_kv_strided(
            p, 0, q_rs, p, 0, k_rs, p, 0, 128, p, 1, p, p, p, p, p, 0, o_rs, p, 1, N, 4, None)
    assert strided(q_rs=64) == 1 and b"row strides >= 128" in L.t2t_last_error()
    assert strided(o_rs=132) == 1                         # not a multiple of 8 elements
    assert strided(k_rs=1 << 20, N=4096) == 1 and b"4 GiB" in L.t2t_last_error()
    assert L.t2t_resid_merge_inplace_strided(p, 0, 100, p, p, p, p, p, p, p, p, p, 1, 1, 64, 4,
                                            None) == 1
