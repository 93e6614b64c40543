"""Static KV metadata for HIP-graph decode replay.

Mirrors pipeswift/utils/cudagraph.py:9-118.  The captured append reads the
static ``slot_mapping`` buffer, which starts at -1 and is padded with -1
beyond the live batch at every refresh, so padded graph rows never write the
cache (the append skips negative slots).  Refreshes use ``copy_`` and
``fill_``/``zero_``, which are kernels on ROCm, never a memset node.
"""

from __future__ import annotations

import torch

from .metadata import KVCacheInfo


def initialize_graph_kvcacheinfo(max_bsz, max_num_pages, max_num_tokens=None, device="cuda"):
    if max_num_tokens is None:
        max_num_tokens = max_bsz
    s = KVCacheInfo()
    s.page_table = torch.zeros((max_bsz, max_num_pages), dtype=torch.int32, device=device)
    s.slot_mapping = torch.full((max_num_tokens,), -1, dtype=torch.int64, device=device)
    s.actual_lens_q = torch.ones((max_bsz,), dtype=torch.int32, device=device)
    s.actual_lens_kv = torch.zeros((max_bsz,), dtype=torch.int32, device=device)
    s.cu_seqlens_q = torch.arange(max_bsz + 1, dtype=torch.int32, device=device)
    s.seqs_kv_pages = torch.zeros((max_bsz * max_num_pages), dtype=torch.int32, device=device)
    s.seqs_kv_page_indptrs = torch.zeros((max_bsz + 1,), dtype=torch.int32, device=device)
    s.actual_lens_q_cpu = torch.ones((max_bsz,), dtype=torch.int32)
    return s


def slice_kvcache_info(info: KVCacheInfo, bsz, num_tokens=None):
    if num_tokens is None:
        num_tokens = bsz
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
    out.actual_lens_q_cpu = None if info.actual_lens_q_cpu is None else info.actual_lens_q_cpu[:bsz]
    out.actual_lens_kv_cpu = None if info.actual_lens_kv_cpu is None else info.actual_lens_kv_cpu[:bsz]
    out.cu_seqlens_q_cpu = None if info.cu_seqlens_q_cpu is None else info.cu_seqlens_q_cpu[: bsz + 1]
    out.seqs_kv_page_indptrs_cpu = (
        None if info.seqs_kv_page_indptrs_cpu is None else info.seqs_kv_page_indptrs_cpu[: bsz + 1]
    )
    out.k_scale = info.k_scale
    out.v_scale = info.v_scale
    out.cg_bsz = bsz
    return out


def set_graph_kvcacheinfo(static: KVCacheInfo, info: KVCacheInfo, cg_bsz, pad_q_len=1):
    assert info is not None
    bsz, max_pages = info.actual_lens_q.shape[0], info.page_table.shape[1]
    static.page_table[:bsz, :max_pages].copy_(info.page_table, non_blocking=True)
    static.slot_mapping[: info.slot_mapping.shape[0]].copy_(info.slot_mapping, non_blocking=True)
    static.actual_lens_q[:bsz].copy_(info.actual_lens_q, non_blocking=True)
    static.actual_lens_kv[:bsz].copy_(info.actual_lens_kv, non_blocking=True)
    static.cu_seqlens_q[: bsz + 1].copy_(info.cu_seqlens_q, non_blocking=True)
    if bsz != cg_bsz:
        assert bsz < cg_bsz
        static.actual_lens_q[bsz:].fill_(pad_q_len)
        static.slot_mapping[info.slot_mapping.shape[0]:].fill_(-1)
        static.actual_lens_kv[bsz:].zero_()
        static.page_table[bsz:, :max_pages].zero_()
        tail = static.cu_seqlens_q.shape[0] - bsz
        static.cu_seqlens_q[bsz + 1:].copy_(
            static.cu_seqlens_q[bsz]
            + torch.arange(pad_q_len, tail * pad_q_len, pad_q_len, dtype=torch.int32,
                           device=static.cu_seqlens_q.device),
            non_blocking=True,
        )
