"""KV-cache metadata: the slot_mapping / page_table contract of the append.

Mirrors the KV part of pipeswift/utils/metadata.py: ``KVCacheInfo``
(:187-203), ``prepare_kv_info`` (:206-348) and
``derive_kvcache_info_next_decode_step`` (:351-414).  The reference builds
slot_mapping with a Python loop over every token and moves it from pageable
memory; here the per-token work is native (``psk_build_kv_metadata`` in
libpipeswift_kv) and writes into a pinned block that reaches the device in one
asynchronous copy, with the same results (decode context parallel included).

The DCP degree and rank are explicit arguments instead of the reference's
global ``parallel_state`` (mpu.py), so the builder has no distributed
dependency; a caller with a process group passes its own values.

Build extensions: ``KVCacheInfo.k_scale`` / ``v_scale`` carry optional
per-tensor FP8 scales (fp32 device tensors, one element or one per layer).
"""

from __future__ import annotations

from array import array
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from ._lib import check, lib


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


class _PinnedStager:
    """Ring of pinned host blocks that carry one step's metadata to the device
    in a single asynchronous copy.  A block is reused only after the copy that
    read it has completed (an event per block)."""

    def __init__(self, slots: int = 8):
        self.blocks = [None] * slots
        self.events = [None] * slots
        self.next = 0

    def acquire(self, nbytes: int):
        i = self.next
        self.next = (i + 1) % len(self.blocks)
        if self.events[i] is not None:
            self.events[i].synchronize()
            self.events[i] = None
        blk = self.blocks[i]
        if blk is None or blk.numel() < nbytes:
            blk = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, pin_memory=torch.cuda.is_available())
            self.blocks[i] = blk
        return i, blk

    def release(self, i: int, stream) -> None:
        ev = torch.cuda.Event()
        ev.record(stream)
        self.events[i] = ev


_stagers: dict = {}


def _page_ptr(pt, keep):
    """(address, length) of a sequence's int32 page ids without copying when
    they already live in an int32 buffer (array('i'), numpy int32)."""
    if isinstance(pt, array) and pt.typecode == "i":
        addr, n = pt.buffer_info()
        return addr, n
    if isinstance(pt, torch.Tensor):
        pt = pt.cpu().numpy()
    a = np.ascontiguousarray(pt, dtype=np.int32)
    keep.append(a)
    return a.ctypes.data, a.shape[0]


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
    zero-padded int32 page_table [B, max_pages], the int64 slot_mapping over the
    new tokens, and the length arrays.  The per-token work runs natively
    (``psk_build_kv_metadata``) into a pinned block that reaches the device in
    one asynchronous copy; the device tensors are views of that one buffer.
    """
    num_seqs = len(seqs)
    assert num_seqs != 0
    device = torch.device(device)
    keep = []
    ptrs = np.empty(num_seqs, dtype=np.uint64)
    plen = np.empty(num_seqs, dtype=np.int64)
    ntok = np.empty(num_seqs, dtype=np.int64)
    offs = np.empty(num_seqs, dtype=np.int64)
    for i, seq in enumerate(seqs):
        ptrs[i], plen[i] = _page_ptr(kv_page_table[seq.seq_id], keep)
        ntok[i] = len(seq.token_ids)
        offs[i] = seq.offset
    W = int(plen.max())
    T = int((ntok - offs).sum())
    B = num_seqs
    o_pt = 8 * T
    o_cu = o_pt + 4 * B * W
    o_lq = o_cu + 4 * (B + 1)
    o_lk = o_lq + 4 * B
    nbytes = o_lk + 4 * B
    on_gpu = device.type == "cuda"
    stager = _stagers.setdefault(device if on_gpu else "cpu", _PinnedStager())
    slot, blk = stager.acquire(nbytes)
    base = blk.data_ptr()
    got = lib().psk_build_kv_metadata(
        B, ptrs.ctypes.data, plen.ctypes.data, ntok.ctypes.data, offs.ctypes.data, kv_page_size, dcp_deg,
        dcp_rank, dcp_interleave_size, int(bool(is_decode)), W, base + o_pt, base + o_cu, base + o_lq, base + o_lk,
        base, T,
    )
    if got < 0:
        if got == -3:
            raise IndexError(lib().psk_last_error().decode())
        check(int(got), "prepare_kv_info")
    host = blk[:nbytes]
    if on_gpu:
        dev = torch.empty(nbytes, dtype=torch.uint8, device=device)
        dev.copy_(host, non_blocking=True)
        stager.release(slot, torch.cuda.current_stream(device))
    else:
        dev = host.clone()
    slot_mapping = dev[:o_pt].view(torch.int64)
    page_table = dev[o_pt:o_cu].view(torch.int32).view(B, W)
    cu_q = dev[o_cu:o_lq].view(torch.int32)
    lens_q = dev[o_lq:o_lk].view(torch.int32)
    lens_kv = dev[o_lk:nbytes].view(torch.int32)
    # host copies outlive the staging block
    cpu = host[o_cu:nbytes].clone()
    cu_q_cpu = cpu[: 4 * (B + 1)].view(torch.int32)
    lens_q_cpu = cpu[4 * (B + 1): 4 * (2 * B + 1)].view(torch.int32)
    lens_kv_cpu = cpu[4 * (2 * B + 1):].view(torch.int32)

    info = KVCacheInfo(
        kv_cache=(kv_cache[0], kv_cache[1]) if kv_cache is not None else None,
        mla_cache_tensor=mla_cache_tensor,
        page_table=page_table,
        slot_mapping=slot_mapping,
        actual_lens_q=lens_q,
        actual_lens_kv=lens_kv,
        cu_seqlens_q=cu_q,
        actual_lens_q_cpu=lens_q_cpu,
        cu_seqlens_q_cpu=cu_q_cpu,
        actual_lens_kv_cpu=lens_kv_cpu,
    )
    if attention_backend == "flash_mla" and not is_decode:
        info.seqs_kv_pages = page_table.view(-1)
        info.seqs_kv_page_indptrs = torch.arange(0, W * B + 1, max(W, 1), device=device, dtype=torch.int32)
        info.seqs_kv_page_indptrs_cpu = torch.arange(0, W * B + 1, max(W, 1), dtype=torch.int32)
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
    token per sequence at position ``seq.offset``; its slot, and lens_kv + 1
    where this rank owns the token (always without DCP).

    The per-sequence work runs natively (``psk_build_next_decode_metadata``)
    into a pinned block that reaches the device in one asynchronous copy; the
    page table, lens_q and cu_seqlens_q stay those of ``prev``."""
    num_seqs = len(seqs)
    assert num_seqs != 0
    device = torch.device(device)
    keep = []
    ptrs = np.empty(num_seqs, dtype=np.uint64)
    plen = np.empty(num_seqs, dtype=np.int64)
    pos = np.empty(num_seqs, dtype=np.int64)
    for i, seq in enumerate(seqs):
        ptrs[i], plen[i] = _page_ptr(kv_page_table[seq.seq_id], keep)
        pos[i] = seq.offset
    prev_kv = np.ascontiguousarray(prev.actual_lens_kv_cpu.numpy(), dtype=np.int32)
    K = prev_kv.shape[0]
    assert K >= num_seqs, "previous step has fewer sequences"
    B = num_seqs
    # lens_kv keeps all K entries of the previous step, the first B advanced
    # (the reference copies the whole previous array, metadata.py:367-369)
    nbytes = 8 * B + 4 * K
    on_gpu = device.type == "cuda"
    stager = _stagers.setdefault(device if on_gpu else "cpu", _PinnedStager())
    slot, blk = stager.acquire(nbytes)
    base = blk.data_ptr()
    got = lib().psk_build_next_decode_metadata(
        B, ptrs.ctypes.data, plen.ctypes.data, pos.ctypes.data, prev_kv.ctypes.data, kv_page_size, dcp_deg,
        dcp_rank, dcp_interleave_size, base, base + 8 * B,
    )
    if got < 0:
        if got == -3:
            raise IndexError(lib().psk_last_error().decode())
        check(int(got), "derive_kvcache_info_next_decode_step")
    host = blk[:nbytes]
    if K > B:
        host[8 * B + 4 * B:].view(torch.int32).copy_(torch.from_numpy(prev_kv[B:]))
    if on_gpu:
        dev = torch.empty(nbytes, dtype=torch.uint8, device=device)
        dev.copy_(host, non_blocking=True)
        stager.release(slot, torch.cuda.current_stream(device))
    else:
        dev = host.clone()
    lens_kv_cpu = host[8 * B:].clone().view(torch.int32)
    return KVCacheInfo(
        kv_cache=prev.kv_cache,
        mla_cache_tensor=prev.mla_cache_tensor,
        page_table=prev.page_table,
        slot_mapping=dev[: 8 * B].view(torch.int64),
        actual_lens_q=prev.actual_lens_q,
        actual_lens_kv=dev[8 * B:].view(torch.int32),
        cu_seqlens_q=prev.cu_seqlens_q,
        actual_lens_q_cpu=prev.actual_lens_q_cpu,
        cu_seqlens_q_cpu=prev.cu_seqlens_q_cpu,
        actual_lens_kv_cpu=lens_kv_cpu,
        k_scale=prev.k_scale,
        v_scale=prev.v_scale,
    )
