"""Block gather, copy_blocks and the per-tensor FP8 scale, on gfx950 HIP kernels.

None of these has a counterpart in the reference (wsjdsg/PipeSwift):
  * its attention kernels read the paged cache in place through the page table
    (pipeswift/llms/layers/attention.py:189-211), so there is no gather;
  * its prefix cache shares whole pages by refcount and remaps a duplicate page
    instead of copying it (pipeswift/engine/block_manager.py:723-780, 841-877),
    so there is no copy_blocks;
  * its FP8 KV cache uses a fixed scale of 1.0 (pipeswift/utils/fp8_kv.py:1-3).
They follow vLLM's conventions for the same operations and are pinned by the
closed forms in their docstrings.
"""

from __future__ import annotations

import math
import threading

import numpy as np
import torch

from ._lib import check, dtype_code, lib, ptr, stream_handle

FP8_E4M3_MAX = 448.0


# --------------------------------------------------------------------------- #
# gather
# --------------------------------------------------------------------------- #


def _row_len(cache: torch.Tensor) -> int:
    """Elements per slot row; the row (dims 2..) must be contiguous."""
    row = 1
    expect = 1
    for dim in range(cache.ndim - 1, 1, -1):
        assert cache.stride(dim) == expect or cache.shape[dim] == 1, (
            f"cache rows must be contiguous beyond dim 1 (strides {cache.stride()})"
        )
        expect *= cache.shape[dim]
        row *= cache.shape[dim]
    return row


def gather_cache(
    src_cache: torch.Tensor,
    dst: torch.Tensor,
    block_table: torch.Tensor,
    cu_seq_lens: torch.Tensor,
    batch_size: int | None = None,
    seq_starts: torch.Tensor | None = None,
    scale: torch.Tensor | None = None,
    src_cache_v: torch.Tensor | None = None,
    dst_v: torch.Tensor | None = None,
) -> None:
    """Copy each sequence's paged rows into contiguous ``dst`` rows.

    src_cache [num_blocks, block_size, *row] (row contiguous; e.g. the K view
    [P, ps, H, D] of the fused [L, P, 2, ps, H, D] cache), dst [T, *row],
    block_table int32 [B, W], cu_seq_lens int32 [B + 1], seq_starts int32 [B]
    (optional first position gathered per sequence).  For t in
    [cu[b], cu[b+1]) and p = seq_starts[b] + t - cu[b]:
    ``dst[t] = src_cache[block_table[b, p // block_size], p % block_size]``.
    A block id outside the cache, or a p beyond the table row, gives a zero
    row.  With an fp8 cache and a bf16/fp16/fp32 ``dst`` each element is
    ``round(float(q) * scale)`` (scale 1.0 when None).  ``src_cache_v``/``dst_v``
    gather a second cache of the same geometry (V) in the same launch.
    """
    assert src_cache.is_cuda and dst.is_cuda and block_table.is_cuda and cu_seq_lens.is_cuda
    device = src_cache.device
    assert src_cache.ndim >= 3, "src_cache must be [num_blocks, block_size, ...]"
    row = _row_len(src_cache)
    assert dst.ndim >= 2 and math.prod(dst.shape[1:]) == row, "dst rows must match the cache rows"
    assert dst[0].is_contiguous() if dst.shape[0] else True, "dst rows must be contiguous"
    assert block_table.dtype == torch.int32 and block_table.ndim == 2 and block_table.is_contiguous()
    assert cu_seq_lens.dtype == torch.int32 and cu_seq_lens.is_contiguous()
    B = cu_seq_lens.shape[0] - 1 if batch_size is None else int(batch_size)
    assert 0 <= B <= cu_seq_lens.shape[0] - 1 and B <= block_table.shape[0]
    if seq_starts is not None:
        assert seq_starts.dtype == torch.int32 and seq_starts.is_contiguous() and seq_starts.shape[0] >= B
    is_dequant = src_cache.dtype != dst.dtype
    if is_dequant:
        assert src_cache.dtype == torch.float8_e4m3fn, "dtype change is only defined for an fp8 cache"
    else:
        assert scale is None, "scale only applies to an fp8 -> float gather"
    if scale is not None:
        assert scale.dtype == torch.float32 and scale.numel() == 1 and scale.device == device
    if src_cache_v is not None or dst_v is not None:
        assert src_cache_v is not None and dst_v is not None
        assert src_cache_v.shape == src_cache.shape and src_cache_v.stride() == src_cache.stride()
        assert src_cache_v.dtype == src_cache.dtype
        assert dst_v.shape == dst.shape and dst_v.stride() == dst.stride() and dst_v.dtype == dst.dtype
    for t in (dst, block_table, cu_seq_lens, seq_starts, scale, src_cache_v, dst_v):
        assert t is None or t.device == device, "all tensors must share the cache's device"

    status = lib().psk_gather_cache(
        ptr(src_cache), ptr(src_cache_v), ptr(dst), ptr(dst_v), ptr(block_table), ptr(cu_seq_lens),
        ptr(seq_starts), B, block_table.stride(0), dst.shape[0], row, src_cache.shape[1], src_cache.shape[0],
        src_cache.stride(0), src_cache.stride(1), dst.stride(0),
        dtype_code(src_cache.dtype), dtype_code(dst.dtype), ptr(scale), stream_handle(device),
    )
    check(status, "gather_cache")


# --------------------------------------------------------------------------- #
# copy_blocks
# --------------------------------------------------------------------------- #


def validate_block_mapping(mapping: np.ndarray, num_blocks: int) -> None:
    """Snapshot preconditions: ids in range, unique destinations, destinations
    disjoint from sources.  Raises AssertionError."""
    m = np.asarray(mapping, dtype=np.int64).reshape(-1, 2)
    if len(m) == 0:
        return
    bad = np.flatnonzero(((m < 0) | (m >= num_blocks)).any(axis=1))
    assert len(bad) == 0, f"block ids out of range [0, {num_blocks}): {m[bad[:8]].tolist()}"
    assert len(np.unique(m[:, 1])) == len(m), "duplicate destination block"
    clash = np.isin(m[:, 1], m[:, 0])
    assert not clash.any(), f"destination blocks that are also sources: {m[clash, 1][:8].tolist()}"


def _slab(cache: torch.Tensor):
    """(num_layers, layer_stride, block_stride, block_bytes) in bytes for a
    layered cache [L, P, ...] whose (layer, page) slab is contiguous."""
    assert cache.ndim >= 3, "caches for copy_blocks are layered: [num_layers, num_blocks, ...]"
    es = cache.element_size()
    expect = 1
    for dim in range(cache.ndim - 1, 1, -1):
        assert cache.stride(dim) == expect or cache.shape[dim] == 1, (
            f"each (layer, block) slab must be contiguous (strides {cache.stride()})"
        )
        expect *= cache.shape[dim]
    return cache.shape[0], cache.stride(0) * es, cache.stride(1) * es, expect * es


def copy_blocks(caches, block_mapping: torch.Tensor, validate: bool = True) -> None:
    """For every cache, layer l and pair (s, d): ``cache[l, d] = cache[l, s]``.

    ``caches`` is one tensor or a list of layered caches [L, num_blocks, ...]
    (pages on dim 1, the layout CopyEngine takes: the fused GQA cache
    [L, P, 2, ps, H, D] moves K and V together, MLA is [L, P, ps, 576]).
    ``block_mapping`` is int64 [n, 2] of (src, dst) on the host or the device.
    With ``validate`` (default) the mapping is checked on the host -- ids in
    range, unique destinations, no destination that is also a source -- which
    makes the copy a snapshot: every read sees the pre-call contents.  A
    device-resident mapping is then copied to the host for the check; pass
    ``validate=False`` to skip it (out-of-range pairs are still skipped by the
    kernel, overlapping ones race).
    """
    if isinstance(caches, torch.Tensor):
        caches = [caches]
    assert len(caches) > 0
    device = caches[0].device
    assert all(c.is_cuda and c.device == device for c in caches)
    assert block_mapping.dtype == torch.int64 and block_mapping.ndim == 2 and block_mapping.shape[1] == 2
    n = block_mapping.shape[0]
    if n == 0:
        return
    if validate:
        host = block_mapping if not block_mapping.is_cuda else block_mapping.cpu()
        for c in caches:
            validate_block_mapping(host.numpy(), c.shape[1])
    if block_mapping.is_cuda:
        assert block_mapping.device == device
        dev_map = block_mapping.contiguous()
    else:
        dev_map = block_mapping.contiguous().pin_memory().to(device, non_blocking=True)
    stream = stream_handle(device)
    for c in caches:
        layers, layer_stride, block_stride, block_bytes = _slab(c)
        status = lib().psk_copy_blocks(
            ptr(c), layers, layer_stride, block_stride, block_bytes, c.shape[1], ptr(dev_map), n, stream
        )
        check(status, "copy_blocks")
    if not block_mapping.is_cuda:
        # keep the staged copy alive until the kernels that read it have run
        dev_map.record_stream(torch.cuda.current_stream(device))


# --------------------------------------------------------------------------- #
# FP8 per-tensor scale
# --------------------------------------------------------------------------- #

_workspaces: dict = {}
_ws_lock = threading.Lock()


def amax_workspace(device) -> torch.Tensor:
    """Per-device uint32 workspace of the amax kernels (partial maxima).

    Allocate it (``warmup``) before any HIP graph capture; it needs no initial
    contents, so it is reusable inside graphs.  Calls that share it must be
    ordered on one stream (they run on the caller's stream).
    """
    device = torch.device(device)
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    ws = _workspaces.get(device)
    if ws is None:
        with _ws_lock:
            ws = _workspaces.get(device)
            if ws is None:
                assert not torch.cuda.is_current_stream_capturing(), (
                    "allocate the amax workspace (cache_ops.warmup) before graph capture"
                )
                n = int(lib().psk_kv_amax_workspace_len())
                ws = torch.zeros(n, dtype=torch.int32, device=device)
                _workspaces[device] = ws
    return ws


def warmup(device) -> None:
    amax_workspace(device)


def compute_kv_scales(
    key: torch.Tensor,
    value: torch.Tensor | None = None,
    qmax: float = FP8_E4M3_MAX,
    out: torch.Tensor | None = None,
    amax_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-tensor scales ``amax / qmax`` (1.0 for an all-zero tensor) for key
    and value, in one launch; returns float32 [2] (or [1] without value).

    amax = max |x| over the tensor, NaN ignored.  Inputs are [N, ...] with
    contiguous rows (dims 1..), e.g. the strided K/V views of a qkv projection.
    """
    assert key.is_cuda
    device = key.device
    tensors = [key] if value is None else [key, value]
    for t in tensors:
        assert t.device == device and t.dtype in (torch.bfloat16, torch.float16, torch.float32)
        assert t.dtype == key.dtype and t.shape == key.shape
    rows = key.shape[0] if key.ndim else 1
    row_len = math.prod(key.shape[1:]) if key.ndim > 1 else 1
    strides = []
    for t in tensors:
        if t.ndim > 1:
            exp = 1
            for dim in range(t.ndim - 1, 0, -1):
                assert t.stride(dim) == exp or t.shape[dim] == 1, "rows must be contiguous"
                exp *= t.shape[dim]
        strides.append(t.stride(0) if t.ndim else 1)
    k = len(tensors)
    if out is None:
        assert not torch.cuda.is_current_stream_capturing(), "pass `out` when capturing"
        out = torch.empty(k, dtype=torch.float32, device=device)
    assert out.dtype == torch.float32 and out.numel() >= k and out.is_contiguous() and out.device == device
    if amax_out is not None:
        assert amax_out.dtype == torch.float32 and amax_out.numel() >= k and amax_out.device == device
    ws = amax_workspace(device)
    if k == 2 and rows * row_len == 0:
        # Empty tensors have NULL data, and a NULL second tensor means "key
        # only" to the C entry: one single-tensor call per output (scale 1.0).
        for j, t in enumerate(tensors):
            status = lib().psk_kv_amax_scale(
                ptr(t), None, rows, row_len, strides[j], strides[j], dtype_code(key.dtype), float(qmax),
                out.data_ptr() + 4 * j, None if amax_out is None else amax_out.data_ptr() + 4 * j,
                ptr(ws), ws.numel(), stream_handle(device),
            )
            check(status, "compute_kv_scales")
        return out
    status = lib().psk_kv_amax_scale(
        ptr(key), ptr(value), rows, row_len, strides[0], strides[-1], dtype_code(key.dtype), float(qmax),
        ptr(out), ptr(amax_out), ptr(ws), ws.numel(), stream_handle(device),
    )
    check(status, "compute_kv_scales")
    return out
