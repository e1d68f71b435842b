"""MiniMax-H3 path of the SGLang backend mirror (forward_varlen,
integrations/sglang/backend/t2t_attn.py:763-1047, 1209-1413).

CPU: configuration defaults, query-cluster count, budget map, the packed
layout rules and the dense fallbacks (checked against one masked attention
over the whole packed sequence, a different formulation from the per-document
loop).  GPU: the sparse call equals the operator run directly on the
reordered [video | context] sequence with the context pinned, context rows
equal dense attention over every used key, padding rows are zero, and at a
full budget the video rows equal dense attention.
"""
import json
import math

import pytest
import torch

from token2tile_amd.backend import t2t_attn as B

SCALE = 1.0 / math.sqrt(128)


@pytest.fixture(autouse=True)
def _clean_context():
    B.set_backend_config({})
    B.set_forward_context(0, None)
    yield
    B.set_backend_config({})
    B.set_forward_context(0, None)
    B._H3_RUNTIMES.clear()


def _impl(heads=56, layer=0):
    return B.T2TAttentionImpl(heads, 128, False, SCALE, prefix=f"blocks.{layer}.attn.attn")


def _block_diag_ref(q, k, v, bounds):
    """Dense attention of the packed sequence with a block-diagonal mask;
    rows outside every document are zero."""
    T = q.shape[0]
    doc = torch.full((T,), -1, dtype=torch.long)
    for i, (a, b) in enumerate(zip(bounds[:-1], bounds[1:])):
        doc[a:b] = i
    allowed = (doc[:, None] == doc[None, :]) & (doc[:, None] >= 0)
    s = torch.einsum("qhd,khd->hqk", q.double(), k.double()) * SCALE
    s = s.masked_fill(~allowed[None], float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    return torch.einsum("hqk,khd->qhd", p, v.double())


def test_h3_config_defaults_and_overrides():
    cfg = B._h3_config()
    assert cfg["s_frac"] == 0.05 and cfg["dense_prefix"] == 12 and cfg["mask_refresh"] == 1
    assert cfg["cfg_reuse"] is False and cfg["cq"] == "auto" and cfg["ck"] == 2048
    assert cfg["cond_mode"] == "pin" and cfg["video_tokens"] == 0
    assert cfg["step_profile"] == B._WAN_FROZEN_STEP_PROFILE
    B.set_backend_config({"t2t_h3_s_frac": 0.0125, "t2t_mask_refresh": 0,
                          "t2t_step_profile": [1, 2, 3, 4]})
    cfg = B._h3_config()
    assert cfg["s_frac"] == 0.0125 and cfg["mask_refresh"] == 1 and cfg["step_profile"] == (1, 2, 3, 4)
    B.set_backend_config({"t2t_step_profile": [1, 2, 3]})
    with pytest.raises(ValueError, match="4 step and 6 layer"):
        B._h3_config()


def test_h3_query_cluster_count():
    cfg = B._h3_config()
    # about 128 queries per cluster, rounded to a multiple of 4, at least 64
    for used in (98304, 75600, 40000, 8192, 100):
        cq = B._h3_cq(cfg, used)
        assert cq % 4 == 0 and cq >= 64
        if cq > 64:
            assert abs(used / cq - 128) <= 128 * 2 / cq + 1e-9 * used
    assert B._h3_cq(cfg, 98304) == 768
    assert B._h3_cq({"cq": 100}, 98304) == 100


def test_h3_budget_map():
    cfg = B._h3_config()
    used = 98304
    m = B._h3_ns_map(cfg, used)
    assert set(m) == {(w, l) for w in range(4) for l in range(50)}
    base = int(0.05 * used)
    # layers fall into six buckets of 9,8,8,9,8,8 (bucket = layer*6//50)
    sizes = [sum(1 for l in range(50) if min(l * 6 // 50, 5) == g) for g in range(6)]
    assert sizes == [9, 8, 8, 9, 8, 8]
    first = {}
    for l in range(50):
        first.setdefault(l * 6 // 50, l)
    for w in range(4):
        for l in range(50):
            assert m[(w, l)] == m[(w, first[l * 6 // 50])]
    # the product of the two multipliers scales the base budget
    assert abs(m[(0, 0)] - base * 1.574482 * 1.189098) <= 0.5
    assert abs(m[(2, 49)] - base * 0.555188 * 0.537588) <= 0.5
    # clamped to [1, used]
    big = dict(cfg, s_frac=1.0)
    assert max(B._h3_ns_map(big, 1000).values()) == 1000
    tiny = dict(cfg, s_frac=0.0)
    assert min(B._h3_ns_map(tiny, 1000).values()) == 1
    table = [[(w + 1) * 10 + l for l in range(50)] for w in range(4)]
    t = B._h3_ns_map(cfg, 45, table)
    assert t[(0, 0)] == 10 and t[(3, 49)] == 45 and t[(1, 3)] == 23


def test_h3_ns_table_geometry(tmp_path):
    path = tmp_path / "h3.json"
    rows = [[100] * 50 for _ in range(4)]
    path.write_text(json.dumps({"schema": "t2t_ns_table_v1", "heads": 56, "seq_len": 9000,
                                "ns": rows}))
    B.set_backend_config({"t2t_ns_table": str(path)})
    with pytest.raises(ValueError, match="t2t_h3_video_tokens"):
        B._get_h3_runtime(9000, "cpu", heads=28, video_tokens=9000)
    with pytest.raises(ValueError, match="geometry mismatch"):
        B._get_h3_runtime(9100, "cpu", heads=28, video_tokens=8000)
    # within 64 tokens the table is accepted and the operator is built (which
    # needs a GPU device)
    with pytest.raises(ValueError, match="ROCm GPU"):
        B._get_h3_runtime(9050, "cpu", heads=28, video_tokens=8000)


def test_layout_video_tokens():
    lay = {"video": 6000, "video_start": 1000, "video_stop": 7000}
    assert B._h3_video_tokens_from_layout(7000, lay) == 6000
    assert B._h3_video_tokens_from_layout(7100, lay) == 0          # not this document
    assert B._h3_video_tokens_from_layout(7000, dict(lay, video_start=900)) == 0
    assert B._h3_video_tokens_from_layout(7000, dict(lay, video=0)) == 0
    # keyframe condition rows: only the generated tail counts
    cond = dict(lay, video_tail=5000)
    assert B._h3_video_tokens_from_layout(7000, cond) == 5000
    assert B._h3_video_tokens_from_layout(7000, None) == 0
    B.set_forward_context(13, lay)
    assert B._h3_video_tokens_from_layout(7000) == 6000
    assert B.T2TAttentionImpl._current_step() == 13


def test_cond_sparse_rows_partition():
    lay = {"video": 600, "video_tail": 500, "video_start": 100, "video_stop": 900}
    video, (vid, ctx) = B._h3_cond_sparse_rows(900, "cpu", lay)
    assert video == 600 and vid.numel() == 600 and ctx.numel() == 300
    allr = torch.cat((vid, ctx)).sort().values
    assert torch.equal(allr, torch.arange(900))
    assert torch.equal(vid[:100], torch.arange(100, 200))        # keyframe rows
    assert torch.equal(vid[100:], torch.arange(400, 900))        # generated tail
    assert B._h3_cond_sparse_rows(900, "cpu", dict(lay, video_tail=600)) is None
    assert B._h3_cond_sparse_rows(901, "cpu", lay) is None


def _packed(T, H, g, dtype=torch.float32, device="cpu"):
    return [torch.randn(T, H, 128, generator=g).to(device, dtype) for _ in range(3)]


@pytest.mark.parametrize("case", ["heads", "prefix", "no_video"])
def test_dense_fallbacks_match_block_diagonal_attention(case):
    g = torch.Generator().manual_seed(3)
    heads = 8 if case == "heads" else 56
    q, k, v = _packed(150, heads, g)
    bounds = [0, 37, 120, 140]                                     # three documents + padding
    cu = torch.tensor(bounds, dtype=torch.int32)
    impl = _impl(heads)
    if case == "prefix":
        B.set_backend_config({"t2t_h3_video_tokens": 100})
        B.set_forward_context(11, None)                            # dense prefix is 12 steps
    else:
        B.set_forward_context(20, None)                            # video tokens unset, no layout
    out = impl.forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=140)
    ref = _block_diag_ref(q, k, v, bounds)
    assert torch.allclose(out.double(), ref, atol=1e-5)
    assert bool((out[140:] == 0).all())


def test_sparse_path_argument_checks():
    g = torch.Generator().manual_seed(4)
    q, k, v = _packed(64, 56, g)
    cu = torch.tensor([0, 64], dtype=torch.int32)
    B.set_forward_context(20, None)
    B.set_backend_config({"t2t_h3_video_tokens": 40})
    with pytest.raises(ValueError, match="packed used length"):
        _impl().forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=65)
    with pytest.raises(ValueError, match="head sharding"):
        _impl().forward_varlen(q[:, :28], k[:, :28], v[:, :28], cu_seqlens=cu, max_seqlen=64)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
def _h3_call(dev, used, video, T, s_frac, step, seed=0, layout=None, cond="pin"):
    cfg = {"t2t_h3_s_frac": s_frac, "t2t_h3_cond_mode": cond}
    if layout is None:
        cfg["t2t_h3_video_tokens"] = video
    B.set_backend_config(cfg)
    B.set_forward_context(step, layout)
    g = torch.Generator().manual_seed(seed)
    q, k, v = _packed(T, 56, g, torch.bfloat16, dev)
    cu = torch.tensor([0, used], dtype=torch.int32, device=dev)
    return q, k, v, cu


def _sdpa(q, k, v):
    """[Tq, H, D] x [Tk, H, D] -> [Tq, H, D] in fp32."""
    o = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1).float(), k.transpose(0, 1).float(), v.transpose(0, 1).float(), scale=SCALE)
    return o.transpose(0, 1)


def _cos(a, b):
    return float(torch.nn.functional.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0))


@pytest.mark.gpu
def test_h3_sparse_call_matches_direct_operator(dev):
    from token2tile_amd.deploy_step import MaskedStepDeploy
    used, video, T = 6144, 5120, 6200
    context = used - video
    print(f"[h3] direct operator: used={used} video={video}", flush=True)
    q, k, v, cu = _h3_call(dev, used, video, T, 0.05, step=12)
    impl = _impl(layer=3)
    out = impl.forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=used)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == q.dtype
    assert bool((out[used:] == 0).all())
    assert len(impl._h3_states) == 2                              # 56 heads = two 28-head chunks
    # context rows: dense over all used keys
    ctx_ref = _sdpa(q[:context], k[:used], v[:used]).to(q.dtype)
    assert (out[:context].float() - ctx_ref.float()).abs().max() <= 2e-2
    # video rows: the operator on [video | context] with the context pinned
    cq = B._h3_cq(B._h3_config(), used)
    for chunk in range(2):
        h0, h1 = 28 * chunk, 28 * chunk + 28
        qh, kh, vh = (t[:used, h0:h1].transpose(0, 1) for t in (q, k, v))
        qv = qh[:, context:]
        qk = torch.cat((qv, qv[:, :context]), 1).contiguous()
        kk = torch.cat((kh[:, context:], kh[:, :context]), 1).contiguous()
        vv = torch.cat((vh[:, context:], vh[:, :context]), 1).contiguous()
        op = MaskedStepDeploy(28, used, cq, s_frac=0.05, pin_tail=context, device=dev)
        ns = B._h3_ns_map(B._h3_config(), used)[(0, 3)]
        op.ns_t.fill_(ns)
        st = op.init_state(qk, kk, warm_iters=4, seed=3 * 8 + chunk)
        ref = op.step(qk, kk, vv, st)[:, :video].transpose(0, 1)
        assert torch.equal(out[context:used, h0:h1], ref)
        # the state the backend keeps is the operator's updated state
        assert torch.equal(impl._h3_states[chunk]["ck"], st["ck"])


@pytest.mark.gpu
def test_h3_full_budget_is_dense_and_state_persists(dev):
    used, video, T = 4608, 3584, 4608
    context = used - video
    print(f"[h3] full budget: used={used} video={video}", flush=True)
    q, k, v, cu = _h3_call(dev, used, video, T, 1.0, step=12, seed=1)
    impl = _impl(layer=0)
    out = impl.forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=used)
    ref = _sdpa(q, k, v)
    err = (out.float() - ref).abs().max().item()
    print(f"[h3] full budget max-abs {err:.3e}", flush=True)
    assert err <= 2e-2 and _cos(out, ref) >= 0.999
    states = {c: {n: t.clone() for n, t in st.items()} for c, st in impl._h3_states.items()}
    # a later step keeps the states (projections unchanged, centroids updated)
    B.set_forward_context(13, None)
    out2 = impl.forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=used)
    assert _cos(out2, ref) >= 0.999
    for c in states:
        assert torch.equal(impl._h3_states[c]["Uq"], states[c]["Uq"])
    # back at the first sparse step a new request starts from fresh states
    B.set_forward_context(12, None)
    impl.forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=used)
    assert set(impl._h3_states) == {0, 1}


@pytest.mark.gpu
def test_h3_layout_and_sparse_condition_rows(dev):
    used, T = 5120, 5200
    lay = {"video": 4096, "video_tail": 3584, "video_start": 1024, "video_stop": used}
    print(f"[h3] condition rows: used={used} layout={lay}", flush=True)
    # pin mode: the generated tail is the video segment (from the layout)
    q, k, v, cu = _h3_call(dev, used, 0, T, 1.0, step=20, layout=lay)
    out = _impl(layer=7).forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=used)
    ref = _sdpa(q[:used], k[:used], v[:used])
    assert _cos(out[:used], ref) >= 0.999 and bool((out[used:] == 0).all())
    # sparse mode: keyframe rows join the operator's rows
    B._H3_RUNTIMES.clear()
    q, k, v, cu = _h3_call(dev, used, 0, T, 1.0, step=20, layout=lay, cond="sparse")
    impl = _impl(layer=7)
    out = impl.forward_varlen(q, k, v, cu_seqlens=cu, max_seqlen=used)
    assert B._H3_RUNTIMES and next(iter(B._H3_RUNTIMES.values())).video_tokens == 4096
    assert _cos(out[:used], ref) >= 0.999
    err = (out[:used].float() - ref).abs().max().item()
    assert err <= 2e-2
