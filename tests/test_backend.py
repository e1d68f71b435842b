"""SGLang backend mirror: profile resolution, budget schedule, ns tables, CFG
parity bookkeeping and state sanitising on the CPU; the sparse call through
the backend on the GPU (integrations/sglang/backend/t2t_attn.py)."""
import json
import math

import pytest
import torch

from token2tile_amd.backend import t2t_attn as B


def _meta(**kw):
    base = dict(step_index=20, total_steps=50, cache=B.T2TRequestCache())
    base.update(kw)
    return B.T2TAttentionMetadataBuilder().build(**base)


def test_auto_profile_resolution():
    p = B._resolve_profile(_meta(), 75600, 40)
    assert p.name == "wan21_t2v_14b_n75600_t50" and p.cq == 512 and p.ck == 2048
    assert B._resolve_profile(_meta(), 75600, 12).name == "wan21_t2v_1_3b_n75600_t50"
    assert B._resolve_profile(_meta(), 32760, 12).cq == 256
    with pytest.raises(ValueError, match="No built-in"):
        B._resolve_profile(_meta(), 75601, 40)
    with pytest.raises(ValueError, match="No built-in"):
        B._resolve_profile(_meta(total_steps=40), 75600, 40)


def test_named_and_manual_profiles():
    with pytest.raises(ValueError, match="expects"):
        B._resolve_profile(_meta(profile_name="wan21_t2v_n32760_t50"), 75600, 40)
    with pytest.raises(ValueError, match="Unknown"):
        B._resolve_profile(_meta(profile_name="nope"), 75600, 40)
    with pytest.raises(ValueError, match="require t2t_profile='manual'"):
        B._resolve_profile(_meta(ns_base=100), 75600, 40)
    with pytest.raises(ValueError, match="requires ns_base"):
        B._resolve_profile(_meta(profile_name="manual", ns_base=100), 4096, 12)
    m = _meta(profile_name="manual", ns_base=200, dense_prefix_steps=2, cq=32, ck=128,
              step_profile=(1, 1, 1, 1), layer_profile=(1,) * 6, cfg_mult=(1.0, 0.5))
    p = B._resolve_profile(m, 4096, 12)
    assert p.name == "manual" and p.ns_base == 200 and p.cfg_mult == (1.0, 0.5)
    bad = _meta(profile_name="manual", ns_base=5000, dense_prefix_steps=2, cq=32, ck=128,
                step_profile=(1, 1, 1, 1), layer_profile=(1,) * 6, cfg_mult=(1.0, 1.0))
    with pytest.raises(ValueError, match="ns_base"):
        B._resolve_profile(bad, 4096, 12)
    bad_heads = _meta(profile_name="manual", ns_base=50, dense_prefix_steps=2, cq=32, ck=128,
                      step_profile=(1, 1, 1, 1), layer_profile=(1,) * 6, cfg_mult=(1.0, 1.0))
    with pytest.raises(ValueError, match="head count"):
        B._resolve_profile(bad_heads, 4096, 8)


def test_step_windows_and_layer_buckets():
    # windows: steps 0-20, 21-30, 31-40, 41+
    assert [B._step_window(s) for s in (0, 20, 21, 30, 31, 40, 41, 49)] == [0, 0, 1, 1, 2, 2, 3, 3]
    p40 = B._WAN_PROFILES["wan21_t2v_14b_n75600_t50"]
    p12 = B._WAN_PROFILES["wan21_t2v_1_3b_n75600_t50"]
    # six near-equal layer groups: 40 layers -> sizes 7,7,6,7,7,6; 30 layers -> 5 each
    sizes40 = [sum(B._layer_bucket(l, p40) == g for l in range(40)) for g in range(6)]
    assert sizes40 == [7, 7, 6, 7, 7, 6]
    assert [sum(B._layer_bucket(l, p12) == g for l in range(30)) for g in range(6)] == [5] * 6
    with pytest.raises(ValueError):
        B._layer_factor(40, p40)


def test_ns_map_values():
    p = B._WAN_PROFILES["wan21_t2v_14b_n75600_t50"]
    m = B._ns_map(p, 75600)
    assert len(m) == 4 * 40 * 2
    # hand-evaluated: round(2424 * 1.574482 * 1.189098) = round(4538.2)
    assert m[(0, 0, 0)] == 4538 and m[(0, 0, 1)] == 4538
    # round(2424 * 0.555188 * 0.537588) = round(723.47), last layer group
    assert m[(2, 39, 1)] == 723
    p12 = B._WAN_PROFILES["wan21_t2v_n32760_t50"]
    # layer 10 of 30 is in group 2: round(1050 * 0.884428 * 1.278643) = round(1187.4)
    assert B._ns_map(p12, 32760)[(3, 10, 0)] == 1187
    # clamping to [1, N]
    tiny = B.T2TProfile("t", 12, 100, 50, 100, 0, 4, 8, (5.0, 1.0, 1e-9, 1.0), (1.0,) * 6)
    mt = B._ns_map(tiny, 100)
    assert mt[(0, 0, 0)] == 100 and mt[(2, 0, 0)] == 1


def test_ns_table(tmp_path):
    rows = [[10 + w * 40 + l for l in range(30)] for w in range(4)]
    path = tmp_path / "ns.json"
    path.write_text(json.dumps({"schema": "t2t_ns_table_v1", "heads": 12, "seq_len": 4096,
                                "ns": rows}))
    got, digest, header = B._load_ns_table(str(path), expected_layers=30, max_ns=4096)
    assert got[1][3] == 53 and len(digest) == 64 and header["heads"] == 12
    p = B._WAN_PROFILES["wan21_t2v_1_3b_n75600_t50"]
    m = B._ns_map(p, 4096, got)
    assert m[(1, 3, 0)] == m[(1, 3, 1)] == 53  # cfg_mult is not applied to exact tables
    path.write_text(json.dumps({"schema": "other", "ns": rows}))
    with pytest.raises(ValueError, match="schema"):
        B._load_ns_table(str(path), expected_layers=30, max_ns=4096)
    path.write_text(json.dumps({"schema": "t2t_ns_table_v1", "ns": rows[:3]}))
    with pytest.raises(ValueError, match="4x30"):
        B._load_ns_table(str(path), expected_layers=30, max_ns=4096)
    rows[0][0] = 0
    path.write_text(json.dumps({"schema": "t2t_ns_table_v1", "ns": rows}))
    with pytest.raises(ValueError, match="outside"):
        B._load_ns_table(str(path), expected_layers=30, max_ns=4096)


def test_layer_index_from_prefix():
    assert B.T2TAttentionImpl._get_layer_idx("transformer.blocks.17.attn1") == 17
    assert B.T2TAttentionImpl._get_layer_idx("model.transformer_blocks.3.attn") == 3
    assert B.T2TAttentionImpl._get_layer_idx("a.5.attn.inner") == 5
    with pytest.raises(ValueError):
        B.T2TAttentionImpl._get_layer_idx("attn")


def test_impl_rejects_unsupported():
    scale = 1 / math.sqrt(128)
    with pytest.raises(ValueError, match="causal"):
        B.T2TAttentionImpl(12, 128, True, scale, prefix="blocks.0.attn")
    with pytest.raises(ValueError, match="128"):
        B.T2TAttentionImpl(12, 64, False, scale, prefix="blocks.0.attn")
    with pytest.raises(ValueError, match="grouped"):
        B.T2TAttentionImpl(12, 128, False, scale, num_kv_heads=4, prefix="blocks.0.attn")
    with pytest.raises(ValueError, match="scale"):
        B.T2TAttentionImpl(12, 128, False, 0.5, prefix="blocks.0.attn")


def test_backend_class_surface():
    assert B.T2TAttentionBackend.get_supported_head_sizes() == [128]
    assert B.T2TAttentionBackend.get_impl_cls() is B.T2TAttentionImpl
    assert B.T2TAttentionBackend.get_metadata_cls() is B.T2TAttentionMetadata
    assert B.T2TAttentionBackend.get_builder_cls() is B.T2TAttentionMetadataBuilder


def test_sanitize_state():
    prev = {"ck": torch.ones(2, 4, 3), "cq": torch.ones(2, 4, 3)}
    ck = torch.randn(2, 4, 3)
    ck[0, 1] = float("nan")
    ck[1, 2] = 0.0
    ck[1, 3, 0] = float("inf")
    st = {"ck": ck.clone(), "cq": torch.full((2, 4, 3), 2.0)}
    B._sanitize_state(st, prev)
    for h, c in ((0, 1), (1, 2), (1, 3)):
        assert torch.equal(st["ck"][h, c], torch.ones(3))
    assert torch.equal(st["ck"][0, 0], ck[0, 0]) and torch.equal(st["ck"][1, 0], ck[1, 0])
    assert torch.equal(st["cq"], torch.full((2, 4, 3), 2.0))


# ---------------------------------------------------------------------------
# GPU: the call through the backend equals the operator's call
# ---------------------------------------------------------------------------
def _manual_meta(step, cache, **kw):
    return _meta(step_index=step, cache=cache, profile_name="manual", ns_base=300,
                 dense_prefix_steps=2, cq=32, ck=2048, step_profile=(1.0, 1.0, 1.0, 1.0),
                 layer_profile=(1.0,) * 6, cfg_mult=(1.0, 0.75), **kw)


@pytest.mark.gpu
def test_backend_forward_matches_operator(dev):
    from token2tile_amd import deploy_step
    H, N, D = 12, 4096, 128
    g = torch.Generator(device="cpu").manual_seed(7)
    qkv = [torch.randn(1, N, H, D, generator=g).to(dev, torch.bfloat16) for _ in range(3)]
    impl = B.T2TAttentionImpl(H, D, False, 1 / math.sqrt(D), prefix="blocks.3.attn1")
    cache = B.T2TRequestCache()

    # dense prefix step: plain attention
    out0 = impl.forward(*qkv, _manual_meta(0, cache))
    ref0 = B._dense_attention(*qkv, 1 / math.sqrt(D))
    assert torch.allclose(out0.float(), ref0.float(), atol=2e-2)

    # sparse steps: cond + uncond branch, then the next step
    outs = [impl.forward(*qkv, _manual_meta(s, cache)) for s in (2, 2, 3)]
    assert cache.call_counts[(2, 3)] == 2 and set(cache.states) == {(3, 0), (3, 1)}
    with pytest.raises(RuntimeError, match="more than two"):
        impl.forward(*qkv, _manual_meta(2, cache))

    # the same sequence straight through the operator
    op = deploy_step.MaskedStepDeploy(H, N, 32, C=2048, D=D, s_frac=300 / N, mask_refresh=4,
                                      cfg_reuse=True, device=dev)
    q, k, v = (t[0].transpose(0, 1).contiguous() for t in qkv)
    states = {}
    for (s, par), o in zip(((2, 0), (2, 1), (3, 0)), outs):
        op.set_cfg_call(par, 3, s)
        op.ns_t.fill_(300 if par == 0 else 225)
        if par not in states:
            states[par] = op.init_state(q, k, warm_iters=4, seed=3 * 2 + par)
        ref = op.step(q, k, v, states[par])
        got = o[0].transpose(0, 1)
        assert got.shape == ref.shape and torch.equal(got, ref)
    torch.cuda.synchronize()
