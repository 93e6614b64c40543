"""Paged KV append for MHA/GQA and the MLA latent cache, on gfx950 HIP kernels.

Drop-in for pipeswift/utils/triton_kernels/reshape_and_cache.py: same function
names (the ``triton_*`` names are kept as aliases so callers need no edit), same
argument meaning, same asserts.  The work runs in ``psk_reshape_and_cache`` /
``psk_concat_and_cache_mla`` of libpipeswift_kv.so on the caller's current
stream; nothing is allocated and nothing synchronizes, so both calls can be
captured into a HIP graph exactly like the reference's decode path
(llm.py:462-470).

Build extensions over the reference (all default to the reference's behaviour):
  * ``k_scale`` / ``v_scale`` / ``scale``: optional 1-element fp32 device
    tensors.  For an fp8 cache the stored byte is
    e4m3fn(clamp(x / scale, -448, 448)); with no scale it is the reference's
    scale-1.0 branch (reshape_and_cache.py:66-77).
  * an fp8 MLA cache (the reference rejects FP8 for MLA, arguments.py:459-468).
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check, dtype_code, lib, ptr, stream_handle

FP8_E4M3_MAX = 448.0


def _check_scale(scale, device, name):
    if scale is None:
        return
    assert scale.is_cuda and scale.device == device, f"{name} must live on {device}"
    assert scale.dtype == torch.float32 and scale.numel() == 1, f"{name} must be one float32 element"


def _check_slots(slot_mapping, num_rows, device):
    assert slot_mapping.dtype == torch.int64, "slot_mapping must be int64 (metadata.py builds it with array('q'))"
    assert slot_mapping.ndim == 1 and slot_mapping.is_contiguous(), "slot_mapping must be a contiguous 1-D tensor"
    assert slot_mapping.device == device, "slot_mapping must live on the cache's device"
    # The reference launches one program per slot_mapping entry and reads that
    # token's row (reshape_and_cache.py:31,43,114); a shorter key would be read
    # past its end.
    assert slot_mapping.shape[0] <= num_rows, (
        f"slot_mapping has {slot_mapping.shape[0]} entries but the input has {num_rows} tokens"
    )


def reshape_and_cache_flash(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> None:
    """key/value [N, H, D] -> key_cache/value_cache [num_blocks, block_size, H, D].

    reshape_and_cache.py:83-135.  Token t goes to
    ``cache[slot // block_size, slot % block_size]`` for ``slot =
    slot_mapping[t] >= 0``; negative slots (graph padding, foreign DCP tokens)
    are skipped.  Only ``key.stride(0)``/``value.stride(0)`` are used: each
    token's [H, D] is read as one flat row, as the reference does.
    """
    assert key.ndim == 3 and value.ndim == 3
    assert key_cache.ndim == 4 and value_cache.ndim == 4
    assert key.is_cuda and value.is_cuda and slot_mapping.is_cuda

    num_heads = key.shape[1]
    head_size = key.shape[2]
    assert value.shape[1] == num_heads
    assert value.shape[2] == head_size
    assert key_cache.shape[2] == num_heads
    assert key_cache.shape[3] == head_size
    assert value_cache.shape[2] == num_heads
    assert value_cache.shape[3] == head_size

    is_fp8 = key_cache.dtype == torch.float8_e4m3fn
    assert is_fp8 or key_cache.dtype == key.dtype, (
        f"kv cache dtype {key_cache.dtype} does not match key dtype {key.dtype}"
    )
    assert value_cache.dtype == key_cache.dtype
    assert value.dtype == key.dtype

    # The reference addresses V with key_cache's block, page and head strides
    # and value_cache's dim stride (reshape_and_cache.py:55-60, 121-127).  With
    # differing strides that writes outside value_cache, so it is rejected here.
    assert value_cache.stride()[:3] == key_cache.stride()[:3], (
        "value_cache must share key_cache's block/page/head strides "
        f"({value_cache.stride()[:3]} vs {key_cache.stride()[:3]})"
    )
    device = key_cache.device
    assert key.device == device and value.device == device and value_cache.device == device
    _check_slots(slot_mapping, min(key.shape[0], value.shape[0]), device)
    if not is_fp8:
        assert k_scale is None and v_scale is None, "k_scale/v_scale only apply to an fp8 cache"
    _check_scale(k_scale, device, "k_scale")
    _check_scale(v_scale, device, "v_scale")

    kc = key_cache.stride()
    vc = (kc[0], kc[1], kc[2], value_cache.stride(3))
    n = slot_mapping.shape[0]
    status = lib().psk_reshape_and_cache(
        ptr(key), ptr(value), ptr(key_cache), ptr(value_cache), ptr(slot_mapping),
        n, num_heads, head_size, key_cache.shape[1], key_cache.shape[0],
        key.stride(0), value.stride(0), _lib.i64_array(kc), _lib.i64_array(vc),
        dtype_code(key.dtype), dtype_code(key_cache.dtype), ptr(k_scale), ptr(v_scale),
        stream_handle(device),
    )
    check(status, "reshape_and_cache_flash")


def reshape_and_cache_flash_amax(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    scales_out: torch.Tensor | None = None,
    amax_out: torch.Tensor | None = None,
    qmax: float = 448.0,
) -> torch.Tensor:
    """The FP8 append with per-tensor scales taken from this step's own K and
    V: the cache bytes and scales of ``cache_ops.compute_kv_scales(key,
    value)`` followed by ``reshape_and_cache_flash(..., k_scale=scales[0:1],
    v_scale=scales[1:2])``, in two launches for decode-sized batches (the
    append's waves finish the amax themselves) and three otherwise.  The
    reference appends with scale 1.0 (fp8_kv.py:1-3, 75-77).  Returns float32
    [2] (``scales_out`` when given), [k_scale, v_scale]."""
    from . import cache_ops

    assert key.ndim == 3 and value.ndim == 3 and key_cache.ndim == 4 and value_cache.ndim == 4
    assert key.is_cuda and value.is_cuda and slot_mapping.is_cuda
    num_heads, head_size = key.shape[1], key.shape[2]
    assert value.shape[1:] == key.shape[1:] and key_cache.shape[2:] == (num_heads, head_size)
    assert value_cache.shape[2:] == (num_heads, head_size)
    assert key_cache.dtype == torch.float8_e4m3fn and value_cache.dtype == key_cache.dtype, "the cache must be fp8"
    assert key.dtype in (torch.bfloat16, torch.float16, torch.float32) and value.dtype == key.dtype
    assert key.shape[0] == value.shape[0] == slot_mapping.shape[0], "one slot per K/V row"
    for t in (key, value):  # a token's [H, D] is one flat row
        assert t.stride(2) == 1 and (t.stride(1) == head_size or num_heads == 1)
    assert value_cache.stride()[:3] == key_cache.stride()[:3], "value_cache must share key_cache's strides"
    device = key_cache.device
    assert key.device == device and value.device == device and value_cache.device == device
    _check_slots(slot_mapping, key.shape[0], device)
    if scales_out is None:
        assert not torch.cuda.is_current_stream_capturing(), "pass `scales_out` when capturing"
        scales_out = torch.empty(2, dtype=torch.float32, device=device)
    assert scales_out.dtype == torch.float32 and scales_out.numel() >= 2 and scales_out.is_contiguous()
    assert scales_out.device == device
    if amax_out is not None:
        assert amax_out.dtype == torch.float32 and amax_out.numel() >= 2 and amax_out.device == device
    ws = cache_ops.amax_workspace(device)
    kc = key_cache.stride()
    vc = (kc[0], kc[1], kc[2], value_cache.stride(3))
    status = lib().psk_reshape_and_cache_amax(
        ptr(key), ptr(value), ptr(key_cache), ptr(value_cache), ptr(slot_mapping),
        key.shape[0], num_heads, head_size, key_cache.shape[1], key_cache.shape[0],
        key.stride(0), value.stride(0), _lib.i64_array(kc), _lib.i64_array(vc),
        dtype_code(key.dtype), float(qmax), ptr(scales_out), ptr(amax_out), ptr(ws), ws.numel(),
        stream_handle(device),
    )
    check(status, "reshape_and_cache_flash_amax")
    return scales_out


def reshape_and_cache_flash_diffkv(
    key: torch.Tensor,
    value: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    scale: torch.Tensor | None = None,
) -> None:
    """MLA concat: key [N, H, Dk] and value [N, H, Dv] into kv_cache [P, ps, H, Dk+Dv].

    reshape_and_cache.py:191-229.  The cache row of a slot receives the
    token's H*Dk key elements followed by its H*Dv value elements, both read
    flat from the token's row start (the reference's ``tile_pos`` addressing,
    :161-188; for H == 1, the MLA case, that is exactly [kv_c | k_pe]).
    """
    assert key.ndim == 3 and value.ndim == 3
    assert kv_cache.ndim == 4
    assert key.is_cuda and value.is_cuda and kv_cache.is_cuda and slot_mapping.is_cuda

    num_heads = key.shape[1]
    head_size_k = key.shape[2]
    head_size_v = value.shape[2]
    assert value.shape[1] == num_heads
    assert kv_cache.shape[2] == num_heads
    assert kv_cache.shape[3] == head_size_k + head_size_v

    is_fp8 = kv_cache.dtype == torch.float8_e4m3fn
    assert is_fp8 or kv_cache.dtype == key.dtype, (
        f"kv cache dtype {kv_cache.dtype} does not match key dtype {key.dtype}"
    )
    assert value.dtype == key.dtype
    device = kv_cache.device
    assert key.device == device and value.device == device
    _check_slots(slot_mapping, min(key.shape[0], value.shape[0]), device)
    if not is_fp8:
        assert scale is None, "scale only applies to an fp8 cache"
    _check_scale(scale, device, "scale")

    n = slot_mapping.shape[0]
    status = lib().psk_concat_and_cache_mla(
        ptr(key), ptr(value), ptr(kv_cache), ptr(slot_mapping), n,
        num_heads * head_size_k, num_heads * head_size_v, key.stride(0), value.stride(0),
        kv_cache.shape[1], kv_cache.shape[0], kv_cache.stride(0), kv_cache.stride(1),
        dtype_code(key.dtype), dtype_code(kv_cache.dtype), ptr(scale), stream_handle(device),
    )
    check(status, "reshape_and_cache_flash_diffkv")


# The reference's names, so `from ... import triton_reshape_and_cache_flash`
# keeps working after the module swap.
triton_reshape_and_cache_flash = reshape_and_cache_flash
triton_reshape_and_cache_flash_diffkv = reshape_and_cache_flash_diffkv
