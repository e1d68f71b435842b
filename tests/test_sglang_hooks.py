"""SGLang-side hooks (integrations/sglang/token2tile_sglang.patch): the gfx950
resolver gate, the denoising metadata branch and the H3 layout record, which
the H3 path then reads."""
import pytest
import torch

from token2tile_amd.backend import sglang_hooks as S
from token2tile_amd.backend import t2t_attn as B


class _Platform:
    def __init__(self, arch):
        self.arch = arch

    def get_device_arch(self):
        return self.arch


def test_resolver_gates_on_gfx950():
    assert S.resolve_backend(arch="gfx950") == S.BACKEND_PATH
    assert S.resolve_backend(_Platform("gfx950:sramecc+:xnack-")) == S.BACKEND_PATH
    for bad in ("gfx942", "gfx90a", "", None):
        with pytest.raises(ValueError, match="gfx950"):
            S.resolve_backend(_Platform(bad))
    # the path names an importable class with the backend surface
    mod, cls = S.BACKEND_PATH.rsplit(".", 1)
    backend = getattr(__import__(mod, fromlist=[cls]), cls)
    assert backend is B.T2TAttentionBackend
    assert backend.get_impl_cls() is B.T2TAttentionImpl


def test_denoising_metadata_keeps_one_cache_per_request():
    builder = B.T2TAttentionMetadataBuilder()
    cfg = {"t2t_profile": "manual", "t2t_ns_base": 300, "t2t_dense_prefix_steps": 2,
           "t2t_cq": 32, "t2t_ck": 2048, "t2t_step_profile": [1, 1, 1, 1],
           "t2t_layer_profile": [1] * 6, "t2t_cfg_mult": [1.0, 0.5], "t2t_mask_refresh": 2}
    extra = {}
    steps = list(range(20))
    m0 = S.build_denoising_metadata(builder, cfg, extra, 0, steps)
    m5 = S.build_denoising_metadata(builder, cfg, extra, 5, steps)
    assert m0.cache is m5.cache is extra["t2t_cache"]
    assert (m5.step_index, m5.total_steps, m5.profile_name, m5.ns_base) == (5, 20, "manual", 300)
    assert m5.cfg_mult == (1.0, 0.5) and m5.mask_refresh == 2 and m5.cfg_reuse is True
    other = {}
    assert S.build_denoising_metadata(builder, cfg, other, 0, steps).cache is not m0.cache
    d = S.build_denoising_metadata(builder, None, {}, 3, steps)
    assert d.profile_name == "auto" and d.ns_base is None and d.warm_iters == 4
    with pytest.raises(ValueError, match="timesteps"):
        S.build_denoising_metadata(builder, cfg, {}, 0, None)


def test_h3_layout_record_drives_the_varlen_rules():
    # packed [text 40 | keyframes 100 | audio 60 | generated video 500]
    text = torch.arange(0, 40)
    key = torch.arange(40, 140)
    audio = torch.arange(140, 200)
    gen = torch.arange(200, 700)
    lay = S.minimax_h3_layout(torch.cat((key, gen)), audio, text)
    assert lay == {"video_tail": 500, "video": 600, "video_start": 40, "video_stop": 700,
                   "audio": 60, "text_rows": 40}
    assert B._h3_video_tokens_from_layout(700, lay) == 500
    video, (vid, ctx) = B._h3_cond_sparse_rows(700, "cpu", lay)
    assert video == 600
    assert torch.equal(vid, torch.cat((key, gen)))
    assert torch.equal(ctx, torch.cat((text, audio)))
    # no keyframes: video follows the audio and the whole image segment is the tail
    lay2 = S.minimax_h3_layout(gen, audio, text)
    assert lay2["video_tail"] == lay2["video"] == 500
    assert B._h3_video_tokens_from_layout(700, lay2) == 500
    assert B._h3_cond_sparse_rows(700, "cpu", lay2) is None
    empty = S.minimax_h3_layout(torch.empty(0, dtype=torch.long), audio, text)
    assert empty["video"] == 0 and empty["video_start"] == -1


@pytest.mark.gpu
def test_resolver_on_this_device(dev):
    assert S.device_arch() == "gfx950"
    assert S.resolve_backend() == S.BACKEND_PATH


def _old_side(patch_text):
    """Files holding each hunk's old-side lines at the hunk's old start line
    (filler elsewhere): enough for `git apply` to check the hunk headers."""
    import re
    files, cur = {}, None
    lines = patch_text.splitlines()
    i = 0
    while i < len(lines):
        ln = lines[i]
        if ln.startswith("--- a/"):
            cur = ln[6:]
            files.setdefault(cur, {})
        m = re.match(r"@@ -(\d+),(\d+) \+\d+,\d+ @@", ln)
        if m:
            at, n = int(m.group(1)), int(m.group(2))
            i += 1
            while n:
                body = lines[i]
                if body[:1] in (" ", "-") or body == "":
                    files[cur][at] = body[1:]
                    at += 1
                    n -= 1
                i += 1
            continue
        i += 1
    out = {}
    for path, rows in files.items():
        last = max(rows) + 5
        out[path] = "\n".join(rows.get(r, f"# filler {r}") for r in range(1, last + 1)) + "\n"
    return out


def test_rocm_patch_applies_and_calls_existing_hooks(tmp_path):
    """The ROCm patch beside the backend parses, applies hunk-for-hunk to its
    own context, adds the T2T_ATTN enum member the backend's get_enum names,
    and only calls hooks this module defines."""
    import pathlib
    import re
    import subprocess
    root = pathlib.Path(S.__file__).parent / "sglang"
    patch = root / "token2tile_rocm.patch"
    text = patch.read_text()
    for path, body in _old_side(text).items():
        f = tmp_path / path
        f.parent.mkdir(parents=True, exist_ok=True)
        f.write_text(body)
    subprocess.run(["git", "init", "-q", str(tmp_path)], check=True)
    subprocess.run(["git", "-C", str(tmp_path), "apply", str(patch)], check=True)
    iface = (tmp_path / "python/sglang/multimodal_gen/runtime/platforms/interface.py").read_text()
    assert "    T2T_ATTN = enum.auto()" in iface
    sargs = (tmp_path / "python/sglang/multimodal_gen/runtime/server_args/server_args.py").read_text()
    # any config that is not already an addict.Dict (None included) is wrapped
    assert "        elif not isinstance(self.attention_backend_config, addict.Dict):" in sargs
    assert "            self.attention_backend_config = addict.Dict(self.attention_backend_config)" in sargs
    assert getattr(B.T2TAttentionBackend.get_enum(), "name", "T2T_ATTN") == "T2T_ATTN"
    assert B.AttentionBackendEnum.T2T_ATTN is B.T2TAttentionBackend.get_enum()
    called = set(re.findall(r"from token2tile_amd\.backend\.sglang_hooks import (\w+)", text))
    assert called == {"build_denoising_metadata", "minimax_h3_layout"}
    for name in called:
        assert callable(getattr(S, name))
    # the apply script pins the SGLang commit the context lines come from
    script = (root / "apply.sh").read_text()
    assert "880ab72f34ead8f39544c7c7e08edbd443964a1f" in script
    assert "token2tile_rocm.patch" in script
