"""KV-cache metadata: the slot_mapping / page_table contract of the append.

Mirrors the KV part of pipeswift/utils/metadata.py: ``KVCacheInfo``
(:187-203), ``prepare_kv_info`` (:206-348) and
``derive_kvcache_info_next_decode_step`` (:351-414).  The reference builds
slot_mapping with a Python loop over every token; here each sequence's slots
are one vectorized numpy expression over its positions, with the same
results (decode context parallel included).

The DCP degree and rank are explicit arguments instead of the reference's
global ``parallel_state`` (mpu.py), so the builder has no distributed
dependency; a caller with a process group passes its own values.

Build extensions: ``KVCacheInfo.k_scale`` / ``v_scale`` carry optional
per-tensor FP8 scales (fp32 device tensors, one element or one per layer).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch


@dataclass
class KVCacheInfo:
    kv_cache: Tuple[torch.Tensor, torch.Tensor] = None
    page_table: torch.Tensor = None
    slot_mapping: torch.Tensor = None
    actual_lens_q: torch.Tensor = None
    actual_lens_kv: torch.Tensor = None
    cu_seqlens_q: torch.Tensor = None

    seqs_kv_pages: torch.Tensor = None
    seqs_kv_page_indptrs: torch.Tensor = None
    mla_cache_tensor: torch.Tensor = None

    actual_lens_q_cpu: torch.Tensor = None
    seqs_kv_page_indptrs_cpu: torch.Tensor = None
    cu_seqlens_q_cpu: torch.Tensor = None
    actual_lens_kv_cpu: torch.Tensor = None

    k_scale: Optional[torch.Tensor] = None
    v_scale: Optional[torch.Tensor] = None


def dcp_local_kv_len(prefix_len: int, dcp_deg: int, dcp_rank: int, dcp_interleave_size: int) -> int:
    """Tokens of a prefix owned by one DCP rank (metadata.py:246-255)."""
    stride = dcp_interleave_size * dcp_deg
    n = prefix_len // stride * dcp_interleave_size
    rem = prefix_len % stride
    if rem >= (dcp_rank + 1) * dcp_interleave_size:
        n += dcp_interleave_size
    elif rem >= dcp_rank * dcp_interleave_size:
        n += rem % dcp_interleave_size
    return n


def build_slot_mapping(page_table_row, start: int, end: int, page_size: int, dcp_deg: int = 1,
                       dcp_rank: int = 0, dcp_interleave_size: int = 1) -> np.ndarray:
    """int64 slots of positions [start, end) of one sequence (metadata.py:272-295).

    dcp_deg == 1: slot = page_table[pos // ps] * ps + pos % ps.
    DCP: a rank owns pos when (pos // interleave) % dcp == rank; its slot is
    page_table[pos // ps] * (ps // dcp) + local_pos % (ps // dcp) with
    local_pos = pos % interleave + pos // (interleave * dcp) * interleave;
    positions of other ranks get -1.
    """
    pt = np.asarray(page_table_row, dtype=np.int64)
    pos = np.arange(start, end, dtype=np.int64)
    if dcp_deg == 1:
        return pt[pos // page_size] * page_size + pos % page_size
    phys = page_size // dcp_deg
    stride = dcp_interleave_size * dcp_deg
    owned = (pos // dcp_interleave_size) % dcp_deg == dcp_rank
    local = pos % dcp_interleave_size + pos // stride * dcp_interleave_size
    slots = pt[pos // page_size] * phys + local % phys
    return np.where(owned, slots, -1).astype(np.int64)


def coalesced_to_cuda(arr_list, device="cuda"):
    """One H2D copy for several small int arrays (impl_utils.py:340-358)."""
    arrs = []
    for a in arr_list:
        if isinstance(a, torch.Tensor):
            a = a.numpy()
        elif not isinstance(a, np.ndarray):
            a = np.array(a, dtype=np.int32)
        arrs.append(a)
    sizes = [a.size for a in arrs]
    big = torch.from_numpy(np.concatenate(arrs)).to(device, non_blocking=True)
    out, off = [], 0
    for n in sizes:
        out.append(big[off: off + n])
        off += n
    return out


def prepare_kv_info(
    seqs: Sequence,
    kv_page_table,
    kv_page_size: int,
    kv_cache,
    mla_cache_tensor,
    dcp_interleave_size: int = 1,
    is_decode: bool = False,
    attention_backend: str = "flash_attn",
    dcp_deg: int = 1,
    dcp_rank: int = 0,
    device="cuda",
) -> KVCacheInfo:
    """Per-step KV metadata for ``seqs`` (metadata.py:206-348).

    Each seq has ``seq_id``, ``token_ids`` and ``offset`` (tokens already in
    the cache); ``kv_page_table[seq_id]`` is its page list.  Produces the
    zero-padded int32 page_table [B, max_pages], int64 slot_mapping over the
    new tokens, and the length arrays.
    """
    num_seqs = len(seqs)
    assert num_seqs != 0
    physical_page_size = kv_page_size if dcp_deg == 1 else kv_page_size // dcp_deg

    lens_q = np.zeros(num_seqs, dtype=np.int32)
    lens_kv = np.zeros(num_seqs, dtype=np.int32)
    max_pages = 0
    for i, seq in enumerate(seqs):
        n_tok = len(seq.token_ids)
        q_len = n_tok - seq.offset
        lens_q[i] = q_len
        if dcp_deg == 1:
            lens_kv[i] = n_tok
        else:
            prefix = n_tok if is_decode and q_len == 1 else seq.offset
            lens_kv[i] = dcp_local_kv_len(prefix, dcp_deg, dcp_rank, dcp_interleave_size)
        max_pages = max(max_pages, len(kv_page_table[seq.seq_id]))
    cu_q = np.zeros(num_seqs + 1, dtype=np.int32)
    np.cumsum(lens_q, out=cu_q[1:])

    page_table = np.zeros((num_seqs, max_pages), dtype=np.int32)
    slot_parts = []
    for i, seq in enumerate(seqs):
        row = np.asarray(kv_page_table[seq.seq_id], dtype=np.int32)
        page_table[i, : len(row)] = row
        slot_parts.append(
            build_slot_mapping(row, seq.offset, len(seq.token_ids), kv_page_size, dcp_deg, dcp_rank,
                               dcp_interleave_size)
        )
    slot_np = np.concatenate(slot_parts).astype(np.int64) if slot_parts else np.zeros(0, np.int64)

    page_table_d, cu_q_d, lens_q_d, lens_kv_d = coalesced_to_cuda(
        [page_table.ravel(), cu_q, lens_q, lens_kv], device
    )
    page_table_d = page_table_d.view(num_seqs, max_pages)
    slot_mapping = torch.from_numpy(slot_np).to(device, non_blocking=True)

    info = KVCacheInfo(
        kv_cache=(kv_cache[0], kv_cache[1]) if kv_cache is not None else None,
        mla_cache_tensor=mla_cache_tensor,
        page_table=page_table_d,
        slot_mapping=slot_mapping,
        actual_lens_q=lens_q_d,
        actual_lens_kv=lens_kv_d,
        cu_seqlens_q=cu_q_d,
        actual_lens_q_cpu=torch.from_numpy(lens_q),
        cu_seqlens_q_cpu=torch.from_numpy(cu_q),
        actual_lens_kv_cpu=torch.from_numpy(lens_kv),
    )
    if attention_backend == "flash_mla" and not is_decode:
        info.seqs_kv_pages = page_table_d.view(-1)
        info.seqs_kv_page_indptrs = torch.arange(
            0, max_pages * num_seqs + 1, max(max_pages, 1), device=device, dtype=torch.int32
        )
        info.seqs_kv_page_indptrs_cpu = torch.arange(
            0, max_pages * num_seqs + 1, max(max_pages, 1), dtype=torch.int32
        )
    return info


def derive_kvcache_info_next_decode_step(
    prev: KVCacheInfo,
    seqs: Sequence,
    kv_page_table,
    kv_page_size: int,
    dcp_interleave_size: int = 1,
    dcp_deg: int = 1,
    dcp_rank: int = 0,
    device="cuda",
) -> KVCacheInfo:
    """Metadata for the next draft decode step (metadata.py:351-414): one new
    token per sequence at position ``seq.offset``."""
    assert len(seqs) != 0
    lens_kv = prev.actual_lens_kv_cpu.numpy().astype(np.int32).copy()
    slots = np.zeros(len(seqs), dtype=np.int64)
    for i, seq in enumerate(seqs):
        s = build_slot_mapping(kv_page_table[seq.seq_id], seq.offset, seq.offset + 1, kv_page_size, dcp_deg,
                               dcp_rank, dcp_interleave_size)[0]
        slots[i] = s
        if s >= 0:
            lens_kv[i] += 1
    slot_mapping = torch.from_numpy(slots).to(device, non_blocking=True)
    lens_kv_cpu = torch.from_numpy(lens_kv)
    return KVCacheInfo(
        kv_cache=prev.kv_cache,
        mla_cache_tensor=prev.mla_cache_tensor,
        page_table=prev.page_table,
        slot_mapping=slot_mapping,
        actual_lens_q=prev.actual_lens_q,
        actual_lens_kv=lens_kv_cpu.to(device, non_blocking=True),
        cu_seqlens_q=prev.cu_seqlens_q,
        actual_lens_q_cpu=prev.actual_lens_q_cpu,
        cu_seqlens_q_cpu=prev.cu_seqlens_q_cpu,
        actual_lens_kv_cpu=lens_kv_cpu,
        k_scale=prev.k_scale,
        v_scale=prev.v_scale,
    )
