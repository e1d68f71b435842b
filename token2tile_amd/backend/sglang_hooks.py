"""The three SGLang-side hooks of the Token2Tile integration, for ROCm/gfx950.

Counterpart of ``integrations/sglang/token2tile_sglang.patch``:

* ``resolve_backend`` - the attention-backend resolver (patch:98-115 gates on
  SM90; this one gates on a gfx950 device, i.e. MI355X / MI350X);
* ``build_denoising_metadata`` - the denoising-stage metadata branch
  (patch:57-86): one ``T2TRequestCache`` per request in ``batch.extra``, the
  ``t2t_*`` keys of ``attention_backend_config`` mapped onto the builder;
* ``minimax_h3_layout`` - the packed-layout record the MiniMax-H3 DiT publishes
  on the forward context (patch:19-38), read by the H3 ``forward_varlen`` path.

SGLang is not a dependency: each hook takes the objects SGLang would pass in
(the platform, the builder, the batch's ``extra`` dict, the position tensors),
so it is called from a few lines added to SGLang's own files.
"""
from __future__ import annotations

from typing import Any

import torch

BACKEND_PATH = "token2tile_amd.backend.t2t_attn.T2TAttentionBackend"
SUPPORTED_ARCH = "gfx950"


def device_arch(device_index: int = 0) -> str:
    """The gfx architecture of a visible ROCm device ('' without one)."""
    if not torch.cuda.is_available() or torch.version.hip is None:
        return ""
    props = torch.cuda.get_device_properties(device_index)
    return str(getattr(props, "gcnArchName", "")).split(":")[0]


def resolve_backend(platform: Any = None, *, arch: str | None = None) -> str:
    """Dotted path of the backend class, or ValueError on a device the HIP
    kernels were not built for (patch:98-115).  ``arch`` overrides the device
    query (``platform.get_device_arch()`` when the platform has it, else the
    first visible device)."""
    if arch is None:
        getter = getattr(platform, "get_device_arch", None)
        arch = getter() if callable(getter) else device_arch()
    arch = (arch or "").split(":")[0]
    if arch != SUPPORTED_ARCH:
        raise ValueError("Token2Tile kernels require a gfx950 GPU (MI355X / MI350X); "
                         f"this device reports {arch or 'unknown'}.")
    from . import t2t_attn  # noqa: F401 - import now so a broken install fails here
    return BACKEND_PATH


def build_denoising_metadata(builder, attention_backend_config: dict | None,
                             batch_extra: dict, step_index: int, timesteps) -> Any:
    """Metadata of denoising step ``step_index`` (patch:57-86).  The request's
    ``T2TRequestCache`` lives in ``batch_extra['t2t_cache']``, created on the
    first step."""
    if timesteps is None:
        raise ValueError("timesteps must be provided for Token2Tile metadata")
    from .t2t_attn import T2TRequestCache
    cfg = attention_backend_config or {}
    cache = batch_extra.get("t2t_cache")
    if cache is None:
        cache = T2TRequestCache()
        batch_extra["t2t_cache"] = cache
    return builder.build(
        step_index=step_index, total_steps=len(timesteps),
        profile_name=cfg.get("t2t_profile", "auto"), ns_base=cfg.get("t2t_ns_base"),
        dense_prefix_steps=cfg.get("t2t_dense_prefix_steps"), cq=cfg.get("t2t_cq"),
        ck=cfg.get("t2t_ck"), step_profile=cfg.get("t2t_step_profile"),
        layer_profile=cfg.get("t2t_layer_profile"), cfg_mult=cfg.get("t2t_cfg_mult"),
        ns_table=cfg.get("t2t_ns_table"), warm_iters=cfg.get("t2t_warm_iters", 4),
        mask_refresh=cfg.get("t2t_mask_refresh", 4), cfg_reuse=cfg.get("t2t_cfg_reuse", True),
        use_kmm=cfg.get("t2t_use_kmm", True), cache=cache)


def minimax_h3_layout(img_pos: torch.Tensor, audio_pos: torch.Tensor,
                      text_pos: torch.Tensor) -> dict[str, int]:
    """Row ranges of the packed H3 document from the DiT's position index
    tensors (patch:19-38).  ``video_tail`` counts the generated-video rows
    after the last audio row; keyframe condition rows (fl2va) sit before the
    audio and are excluded from it."""
    img = img_pos.detach().reshape(-1).to("cpu")
    audio = audio_pos.detach().reshape(-1).to("cpu")
    tail_from = int(audio.max()) + 1 if audio.numel() else 0
    return {
        "video_tail": int((img >= tail_from).sum()),
        "video": int(img.numel()),
        "video_start": int(img.min()) if img.numel() else -1,
        "video_stop": int(img.max()) + 1 if img.numel() else -1,
        "audio": int(audio.numel()),
        "text_rows": int(text_pos.numel()),
    }
