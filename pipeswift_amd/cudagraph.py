"""Static KV metadata for HIP-graph decode replay.

The interface of pipeswift/utils/cudagraph.py:9-118: the captured decode step
reads fixed buffers (``initialize_graph_kvcacheinfo``), a smaller batch runs
a graph captured for a larger one through views (``slice_kvcache_info``), and
before every replay the buffers take the live step's metadata
(``set_graph_kvcacheinfo``).  The static slot_mapping starts at -1 and is
padded with -1 beyond a padded batch, so padded graph rows never write the
cache (the append skips negative slots).

The refresh is one kernel launch (``psk_refresh_graph_metadata``) where the
reference issues about ten (five copies, four fills and an arange chain for the
cu_seqlens_q tail, cudagraph.py:75-118).  The static fields are views of one
device buffer; the kernel reads the step's device metadata, which
``prepare_kv_info`` already placed in one buffer with one asynchronous copy.
No memset node is involved, so the refresh itself may be captured.
"""

from __future__ import annotations

import torch

from ._lib import check, lib, ptr, stream_handle
from .metadata import KVCacheInfo


def initialize_graph_kvcacheinfo(max_bsz, max_num_pages, max_num_tokens=None, device="cuda"):
    """Static buffers of a captured decode step (cudagraph.py:9-35).

    page_table int32 [max_bsz, max_num_pages] zeros, slot_mapping int64
    [max_num_tokens] of -1, actual_lens_q ones, actual_lens_kv zeros,
    cu_seqlens_q 0..max_bsz, seqs_kv_pages / seqs_kv_page_indptrs zeros.  All
    device fields are views of one allocation (int64 fields first, so every
    view is aligned)."""
    if max_num_tokens is None:
        max_num_tokens = max_bsz
    device = torch.device(device)
    n64 = max_num_tokens
    n32 = max_bsz * max_num_pages + 2 * max_bsz + (max_bsz + 1) + max_bsz * max_num_pages + (max_bsz + 1)
    block = torch.empty(8 * n64 + 4 * n32, dtype=torch.uint8, device=device)
    s = KVCacheInfo()
    s.slot_mapping = block[: 8 * n64].view(torch.int64)
    rest = block[8 * n64:].view(torch.int32)
    o = 0

    def take(n):
        nonlocal o
        t = rest[o: o + n]
        o += n
        return t

    s.page_table = take(max_bsz * max_num_pages).view(max_bsz, max_num_pages)
    s.actual_lens_q = take(max_bsz)
    s.actual_lens_kv = take(max_bsz)
    s.cu_seqlens_q = take(max_bsz + 1)
    s.seqs_kv_pages = take(max_bsz * max_num_pages)
    s.seqs_kv_page_indptrs = take(max_bsz + 1)
    # initial contents (set-up only, outside any graph)
    s.slot_mapping.fill_(-1)
    s.page_table.zero_()
    s.actual_lens_q.fill_(1)
    s.actual_lens_kv.zero_()
    s.cu_seqlens_q.copy_(torch.arange(max_bsz + 1, dtype=torch.int32))
    s.seqs_kv_pages.zero_()
    s.seqs_kv_page_indptrs.zero_()
    s.actual_lens_q_cpu = torch.ones((max_bsz,), dtype=torch.int32)
    return s


def slice_kvcache_info(info: KVCacheInfo, bsz, num_tokens=None):
    """Views of the static buffers for a graph of batch ``bsz`` (cudagraph.py:38-72)."""
    if num_tokens is None:
        num_tokens = bsz

    def head(t, n):
        return None if t is None else t[:n]

    out = KVCacheInfo()
    out.kv_cache = info.kv_cache
    out.mla_cache_tensor = info.mla_cache_tensor
    out.page_table = info.page_table[:bsz]
    out.slot_mapping = info.slot_mapping[:num_tokens]
    out.actual_lens_q = info.actual_lens_q[:bsz]
    out.actual_lens_kv = info.actual_lens_kv[:bsz]
    out.cu_seqlens_q = info.cu_seqlens_q[: bsz + 1]
    out.seqs_kv_pages = info.seqs_kv_pages
    out.seqs_kv_page_indptrs = info.seqs_kv_page_indptrs[: bsz + 1]
    out.actual_lens_q_cpu = head(info.actual_lens_q_cpu, bsz)
    out.actual_lens_kv_cpu = head(info.actual_lens_kv_cpu, bsz)
    out.cu_seqlens_q_cpu = head(info.cu_seqlens_q_cpu, bsz + 1)
    out.seqs_kv_page_indptrs_cpu = head(info.seqs_kv_page_indptrs_cpu, bsz + 1)
    out.k_scale = info.k_scale
    out.v_scale = info.v_scale
    out.cg_bsz = bsz
    return out


def _i32_vec(t, name):
    assert t.dtype == torch.int32 and t.ndim == 1 and t.is_contiguous(), f"{name} must be a contiguous int32 vector"


def set_graph_kvcacheinfo(static: KVCacheInfo, info: KVCacheInfo, cg_bsz, pad_q_len=1):
    """Refresh the static buffers from the step's metadata before a replay
    (cudagraph.py:75-118), in one kernel launch on the current stream.

    Copies page_table[:bsz, :W], slot_mapping[:n], the two length vectors and
    cu_seqlens_q[:bsz + 1]; when bsz != cg_bsz (assert bsz < cg_bsz) pads
    lens_q with pad_q_len, slot_mapping with -1, lens_kv and page_table rows
    [bsz:, :W] with 0, and cu_seqlens_q[bsz + 1:] with cu[bsz] + k * pad_q_len.
    """
    assert info is not None
    bsz, width = info.actual_lens_q.shape[0], info.page_table.shape[1]
    if bsz != cg_bsz:
        assert bsz < cg_bsz
    dev = static.slot_mapping.device
    assert dev.type == "cuda", "graph metadata lives on the GPU"
    for t in (info.page_table, info.slot_mapping, info.actual_lens_q, info.actual_lens_kv, info.cu_seqlens_q,
              static.page_table, static.actual_lens_q, static.actual_lens_kv, static.cu_seqlens_q):
        assert t.device == dev, "static and step metadata must share a device"
    assert info.page_table.dtype == torch.int32 and info.page_table.ndim == 2 and info.page_table.stride(1) == 1
    assert static.page_table.dtype == torch.int32 and static.page_table.ndim == 2 and static.page_table.stride(1) == 1
    assert info.slot_mapping.dtype == torch.int64 and info.slot_mapping.is_contiguous()
    assert static.slot_mapping.dtype == torch.int64 and static.slot_mapping.is_contiguous()
    for t, n in ((info.actual_lens_q, "actual_lens_q"), (info.actual_lens_kv, "actual_lens_kv"),
                 (info.cu_seqlens_q, "cu_seqlens_q"), (static.actual_lens_q, "static actual_lens_q"),
                 (static.actual_lens_kv, "static actual_lens_kv"), (static.cu_seqlens_q, "static cu_seqlens_q")):
        _i32_vec(t, n)
    assert info.actual_lens_kv.shape[0] == bsz and info.cu_seqlens_q.shape[0] >= bsz + 1
    max_bsz = static.actual_lens_q.shape[0]
    assert static.actual_lens_kv.shape[0] == max_bsz and static.cu_seqlens_q.shape[0] == max_bsz + 1
    assert static.page_table.shape[0] == max_bsz
    pt_stride = info.page_table.stride(0) if bsz > 0 else width
    status = lib().psk_refresh_graph_metadata(
        ptr(info.page_table), pt_stride, ptr(info.slot_mapping), ptr(info.actual_lens_q),
        ptr(info.actual_lens_kv), ptr(info.cu_seqlens_q), bsz, width, info.slot_mapping.shape[0],
        ptr(static.page_table), static.page_table.stride(0), static.page_table.shape[1], ptr(static.slot_mapping),
        static.slot_mapping.shape[0], ptr(static.actual_lens_q), ptr(static.actual_lens_kv),
        ptr(static.cu_seqlens_q), max_bsz, cg_bsz, int(pad_q_len), stream_handle(dev),
    )
    check(status, "set_graph_kvcacheinfo")

