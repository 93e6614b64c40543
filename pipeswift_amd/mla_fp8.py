"""FP8 MLA latent cache with one scale per 128-element tile.

The reference stores the MLA latent cache in bf16 only: it rejects FP8 for MLA
models because the MLA reader's FP8 cache is "a different quantization scheme
(per-128-element tiles with scales appended to the cache entry)"
(pipeswift/utils/arguments.py:459-467).  This module writes and reads that
entry, the one FlashMLA reads for an FP8 latent cache:

    [0, 512)     kv_c as E4M3FN, tile j = elements [128j, 128j+128) divided by s_j
    [512, 528)   s_0..s_3 as float32
    [528, 656)   k_pe as bf16, unquantized

with s_j = max(amax_j / 448, 2^-126) and amax_j the tile's max |x| (NaN
ignored).  The sizes generalize to any nope part that is a multiple of 128 and
any even rope part (``entry_bytes``).  The cache is a uint8 tensor
[num_blocks, block_size, entry_bytes] (or with a 1-head axis before the entry).

``concat_and_cache_mla_fp8_tiles`` is the append (the FP8 counterpart of
``reshape_and_cache_flash_diffkv``, reshape_and_cache.py:191-229);
``gather_mla_fp8_tiles`` dequantizes whole sequences into contiguous bf16/f32
rows, as ``cache_ops.gather_cache`` does for the GQA cache.  Both run on the
caller's current stream and allocate nothing.
"""

from __future__ import annotations

import torch

from ._lib import check, dtype_code, lib, ptr, stream_handle

TILE = 128
NOPE_DSV3 = 512
ROPE_DSV3 = 64


def entry_bytes(nope_len: int = NOPE_DSV3, rope_len: int = ROPE_DSV3) -> int:
    """Bytes of one entry: nope_len + 4 * nope_len / 128 + 2 * rope_len."""
    n = int(lib().psk_mla_fp8_tile_entry_bytes(nope_len, rope_len))
    check(n if n < 0 else 0, "mla fp8 entry size")
    return n


def _entries(kv_cache: torch.Tensor) -> torch.Tensor:
    """[P, ps, E] view of a [P, ps, E] or [P, ps, 1, E] uint8 cache."""
    assert kv_cache.dtype in (torch.uint8, torch.float8_e4m3fn), "the tile-scaled FP8 cache is a uint8 tensor"
    if kv_cache.ndim == 4:
        assert kv_cache.shape[2] == 1, "one latent head per entry"
        kv_cache = kv_cache.select(2, 0)
    assert kv_cache.ndim == 3 and kv_cache.stride(2) == 1, "cache must be [num_blocks, block_size, entry_bytes]"
    return kv_cache


def concat_and_cache_mla_fp8_tiles(
    kv_c: torch.Tensor,
    k_pe: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """kv_c [N, nope_len] and k_pe [N, rope_len] (bf16, unit inner stride; k_pe
    may be a column slice of a wider projection) into the entries of
    ``kv_cache`` at ``slot_mapping`` (int64 [N]; negative or out-of-range
    slots are skipped, as in the GQA append)."""
    assert kv_c.is_cuda and k_pe.is_cuda and kv_cache.is_cuda and slot_mapping.is_cuda
    if kv_c.ndim == 3:
        assert kv_c.shape[1] == 1 and k_pe.ndim == 3 and k_pe.shape[1] == 1
        kv_c, k_pe = kv_c.select(1, 0), k_pe.select(1, 0)
    assert kv_c.ndim == 2 and k_pe.ndim == 2 and kv_c.shape[0] == k_pe.shape[0]
    assert kv_c.dtype == torch.bfloat16 and k_pe.dtype == torch.bfloat16, "bf16 latent input"
    assert kv_c.stride(1) == 1 and k_pe.stride(1) == 1, "latent rows must have unit inner stride"
    cache = _entries(kv_cache)
    nope, rope = kv_c.shape[1], k_pe.shape[1]
    assert cache.shape[2] == entry_bytes(nope, rope), (
        f"entry of {cache.shape[2]} bytes, want {entry_bytes(nope, rope)} for nope {nope} + rope {rope}"
    )
    device = cache.device
    assert kv_c.device == device and k_pe.device == device and slot_mapping.device == device
    assert slot_mapping.dtype == torch.int64 and slot_mapping.ndim == 1 and slot_mapping.is_contiguous()
    assert slot_mapping.shape[0] <= kv_c.shape[0]
    st = lib().psk_concat_and_cache_mla_fp8_tiles(
        ptr(kv_c), ptr(k_pe), ptr(cache), ptr(slot_mapping), slot_mapping.shape[0], nope, rope,
        kv_c.stride(0), k_pe.stride(0), cache.shape[1], cache.shape[0], cache.stride(0), cache.stride(1),
        dtype_code(kv_c.dtype), stream_handle(device),
    )
    check(st, "concat_and_cache_mla_fp8_tiles")


def gather_mla_fp8_tiles(
    kv_cache: torch.Tensor,
    dst: torch.Tensor,
    block_table: torch.Tensor,
    cu_seq_lens: torch.Tensor,
    batch_size: int | None = None,
    seq_starts: torch.Tensor | None = None,
    rope_len: int = ROPE_DSV3,
) -> None:
    """dst [T, nope_len + rope_len] (bf16 or f32, rows 16-byte aligned) from the
    entries of each sequence's pages: for t in [cu[b], cu[b+1]) and
    p = seq_starts[b] + t - cu[b], the entry at
    ``block_table[b, p // block_size], p % block_size`` dequantized,
    y_i = round(float(q_i) * s_{i // 128}), rope part converted exactly.  Rows
    with no valid block are zeros; rows at or past cu[batch_size] are left
    untouched."""
    assert kv_cache.is_cuda and dst.is_cuda and block_table.is_cuda and cu_seq_lens.is_cuda
    cache = _entries(kv_cache)
    E = cache.shape[2]
    nope = dst.shape[1] - rope_len
    assert dst.ndim == 2 and nope > 0 and E == entry_bytes(nope, rope_len), (
        f"dst rows of {dst.shape[1]} elements do not fit {E}-byte entries with rope {rope_len}"
    )
    assert dst.stride(1) == 1 and dst.dtype in (torch.bfloat16, torch.float32)
    assert block_table.dtype == torch.int32 and block_table.ndim == 2 and block_table.is_contiguous()
    assert cu_seq_lens.dtype == torch.int32 and cu_seq_lens.is_contiguous()
    B = cu_seq_lens.shape[0] - 1 if batch_size is None else int(batch_size)
    assert 0 <= B <= cu_seq_lens.shape[0] - 1 and B <= block_table.shape[0]
    if seq_starts is not None:
        assert seq_starts.dtype == torch.int32 and seq_starts.is_contiguous() and seq_starts.shape[0] >= B
    device = cache.device
    for t in (dst, block_table, cu_seq_lens, seq_starts):
        assert t is None or t.device == device, "all tensors must share the cache's device"
    st = lib().psk_gather_mla_fp8_tiles(
        ptr(cache), ptr(dst), ptr(block_table), ptr(cu_seq_lens), ptr(seq_starts), B, block_table.stride(0),
        dst.shape[0], nope, rope_len, cache.shape[1], cache.shape[0], cache.stride(0), cache.stride(1),
        dst.stride(0) * dst.element_size(), dtype_code(dst.dtype), stream_handle(device),
    )
    check(st, "gather_mla_fp8_tiles")
