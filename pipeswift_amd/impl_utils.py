"""Thin callers of the append, as the attention layers use them.

Mirrors ``append_kv_cache`` / ``append_mla_kv_cache`` of
pipeswift/utils/impl_utils.py:303-325: early return on an empty batch, the
layer's K/V views of ``kv_cache_info.kv_cache`` (GQA) or the layer of
``mla_cache_tensor`` with a 1-head axis (MLA), and ``kv_cache_info.slot_mapping``.
The optional FP8 scales of ``KVCacheInfo`` (one element, or one per layer)
are passed through.  A uint8 ``mla_cache_tensor`` holds tile-scaled FP8 latent
entries (``mla_fp8``), which the append quantizes itself (no per-tensor scale).
"""

from __future__ import annotations

import torch

from .metadata import KVCacheInfo, coalesced_to_cuda  # noqa: F401  (re-exported, impl_utils.py:340)
from .mla_fp8 import concat_and_cache_mla_fp8_tiles
from .reshape_and_cache import reshape_and_cache_flash, reshape_and_cache_flash_diffkv


def _layer_scale(scale, layer_idx):
    if scale is None:
        return None
    return scale if scale.numel() == 1 else scale[layer_idx: layer_idx + 1]


def append_kv_cache(key, value, kv_cache_info: KVCacheInfo = None, layer_idx: int = 0):
    if key.shape[0] == 0:
        return
    reshape_and_cache_flash(
        key,
        value,
        kv_cache_info.kv_cache[0][layer_idx],
        kv_cache_info.kv_cache[1][layer_idx],
        kv_cache_info.slot_mapping,
        _layer_scale(kv_cache_info.k_scale, layer_idx),
        _layer_scale(kv_cache_info.v_scale, layer_idx),
    )


def append_mla_kv_cache(ckv, kpe, kv_cache_info: KVCacheInfo = None, layer_idx: int = 0):
    if ckv.shape[0] == 0:
        return
    cache = kv_cache_info.mla_cache_tensor[layer_idx]
    if cache.dtype == torch.uint8:
        concat_and_cache_mla_fp8_tiles(ckv, kpe, cache, kv_cache_info.slot_mapping)
        return
    reshape_and_cache_flash_diffkv(
        ckv.unsqueeze(1),
        kpe.unsqueeze(1),
        kv_cache_info.mla_cache_tensor[layer_idx].unsqueeze(2),
        kv_cache_info.slot_mapping,
        _layer_scale(kv_cache_info.k_scale, layer_idx),
    )
