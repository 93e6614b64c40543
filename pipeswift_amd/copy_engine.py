"""DRAM L2 offload transport (swap_blocks) for MI355X.

Drop-in for pipeswift/utils/copy_engine.py: the same ``CopyEngine`` /
``CopyHandle`` / ``page_bytes`` / ``make_dma_views`` surface that
BlockManager calls (block_manager.py:190-209, 288, 462, 534), with the transfer
itself in ``psk_swap_blocks`` of libpipeswift_kv.so instead of a ctypes binding
of cuMemcpyBatchAsync.

What is the same as the reference:
  * one pinned host mirror per GPU cache tensor, shaped like the cache but
    ``l2_num_pages`` deep;
  * int8 ``[num_pages, bytes_per_page]`` views per (cache tensor, layer);
  * runs of pages that advance together on both tiers are coalesced on the
    calling thread (the retire deadline is priced from the run count);
  * transfers are ordered after the work already queued on the caller's
    stream through an event, submitted by one daemon thread onto a dedicated
    stream per direction, and signalled by an event on that stream;
  * page indices are range-checked before anything is enqueued;
  * ``calibrate`` fits the same ``t = descriptors/desc_rate + bytes/bw`` model.

What differs, by design for MI355X:
  * the mirror is allocated with hipHostMalloc (mapped, portable) through the
    library instead of torch's caching pinned allocator, which would round a
    multi-GiB mirror up to the next power of two;
  * two transports: ``"blit"`` (default) moves every (view, page) unit in ONE
    kernel that reads/writes the mapped host mirror directly, so the cost per
    descriptor that dominates the reference (copy_engine.py:15-36) disappears;
    ``"memcpy"`` issues one hipMemcpyAsync per (view, run) on the SDMA engines
    (the reference's batched-descriptor call, cuMemcpyBatchAsync, has a HIP
    counterpart that this GPU's runtime does not export);
  * both streams keep the default priority.
"""

from __future__ import annotations

import ctypes
import os
import queue
import threading
import time
from collections import OrderedDict

import numpy as np
import torch

from . import _lib
from ._lib import check, lib

TRANSPORTS = {"memcpy": _lib.SWAP_MEMCPY, "blit": _lib.SWAP_BLIT}
DEFAULT_TRANSPORT = os.environ.get("PIPESWIFT_AMD_SWAP_TRANSPORT", "blit")
_STAGING_SLOTS = 4
# How long a submitter sleeps after queuing a transfer, so that the copy thread
# takes the GIL and enqueues it (CopyEngine._submit).
GIL_HANDOFF_S = 1e-4

_i64p = ctypes.POINTER(ctypes.c_int64)
_u64p = ctypes.POINTER(ctypes.c_uint64)


# --------------------------------------------------------------------------- #
# Cache tensor layout (copy_engine.py:121-142)
# --------------------------------------------------------------------------- #


def page_bytes(caches):
    """Bytes one page occupies across every layer of every cache tensor."""
    return sum(cache[0, 0].numel() * cache.element_size() * cache.shape[0] for cache in caches)


def make_dma_views(caches, num_pages):
    """Flatten each layer to an int8 [num_pages, page_bytes] view.

    Contiguity is required: consecutive pages of a layer must be consecutive
    bytes so that a run of pages is one byte range.
    """
    views = OrderedDict()
    for cache_idx, cache in enumerate(caches):
        assert cache.shape[1] == num_pages
        assert cache.is_contiguous()
        for layer_idx in range(cache.shape[0]):
            layer = cache[layer_idx].reshape(num_pages, -1).view(torch.int8)
            views[f"{cache_idx}.{layer_idx}"] = layer
    return views


# --------------------------------------------------------------------------- #
# pinned host memory
# --------------------------------------------------------------------------- #


class _HostBuffer:
    """hipHostMalloc'd, device-mapped host memory owned by the library."""

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        check(lib().psk_host_alloc(int(nbytes), ctypes.byref(p)), "psk_host_alloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)

    def tensor(self, dtype, shape) -> torch.Tensor:
        raw = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        return torch.frombuffer(raw, dtype=torch.uint8).view(dtype).view(shape)

    def free(self):
        if self.ptr:
            check(lib().psk_host_free(self.ptr), "psk_host_free")
            self.ptr = None


# --------------------------------------------------------------------------- #
# Transport engine
# --------------------------------------------------------------------------- #


class _TransferParams:
    """One direction's geometry: per-view source/destination bases and bytes
    per page, its stream, and (blit) a ring of pinned staging buffers."""

    def __init__(self, src_views, dst_views, stream, src_limit, dst_limit, max_pages):
        assert list(src_views.keys()) == list(dst_views.keys())
        src_bases, dst_bases, bpb = [], [], []
        for src, dst in zip(src_views.values(), dst_views.values()):
            src_bpb = src.stride(0) * src.element_size()
            assert src_bpb == dst.stride(0) * dst.element_size()
            src_bases.append(src.data_ptr())
            dst_bases.append(dst.data_ptr())
            bpb.append(src_bpb)
        self.src_bases = np.array(src_bases, dtype=np.uint64)
        self.dst_bases = np.array(dst_bases, dtype=np.uint64)
        self.bpb = np.array(bpb, dtype=np.uint64)
        self.num_tensors = len(src_bases)
        self.stream = stream
        self.stream_handle = stream.cuda_stream
        self.src_limit = src_limit
        self.dst_limit = dst_limit
        self.max_pages = max_pages
        self.staging = []
        self.desc_dev = None
        self._slot = 0

    def alloc_staging(self, device):
        nbytes = int(lib().psk_swap_staging_bytes(self.num_tensors, self.max_pages))
        self.staging = [[_HostBuffer(nbytes), None] for _ in range(_STAGING_SLOTS)]
        # page tables are copied here before each blit (stream-ordered reuse)
        self.desc_dev = torch.empty(nbytes, dtype=torch.uint8, device=device)

    def next_staging(self):
        """A staging buffer no in-flight transfer still reads."""
        slot = self.staging[self._slot]
        self._slot = (self._slot + 1) % len(self.staging)
        if slot[1] is not None:
            slot[1].synchronize()
        return slot

    def free(self):
        for buf, _ in self.staging:
            buf.free()
        self.staging = []
        self.desc_dev = None


class CopyHandle:
    def __init__(self, pending=True):
        # None until the copy thread has enqueued the batch; an empty transfer
        # never gets one, hence the flag.
        self.event = None
        self.pending = pending
        self.error = None
        # Set synchronously by _submit: the caller prices deadlines from them.
        self.num_runs = 0
        self.num_pages = 0

    def wait(self):
        """Block until the transfer has landed (copy_engine.py:164-177).  Until
        the copy thread has enqueued the transfer there is no event to wait on;
        the loop sleeps rather than spins, because the copy thread needs the GIL
        to get there and a spin with os.sched_yield keeps holding it."""
        if not self.pending:
            return
        while self.event is None:
            if self.error is not None:
                raise self.error
            time.sleep(GIL_HANDOFF_S)
        self.event.synchronize()


class JoinedCopyHandle:
    """One logical transfer submitted as several CopyHandles on one stream
    (they complete in order).  ``num_runs`` / ``num_pages`` describe the whole
    transfer as one submission would (the caller prices deadlines from them)."""

    def __init__(self, handles, num_runs, num_pages):
        self.handles = list(handles)
        self.num_runs = num_runs
        self.num_pages = num_pages

    @property
    def pending(self):
        return any(h.pending for h in self.handles)

    @property
    def error(self):
        return next((h.error for h in self.handles if h.error is not None), None)

    @property
    def event(self):
        return self.handles[-1].event

    def wait(self):
        for h in self.handles:
            h.wait()


class CopyEngine:
    """Pinned host mirror of the KV cache plus the page mover between tiers.

    Transfers are submitted to one background thread so the scheduler never
    blocks on a runtime call, and run on one dedicated stream per direction so
    they overlap the forward pass.  Each returns a CopyHandle.
    """

    def __init__(self, gpu_caches, gpu_num_pages, l2_num_pages, transport=None, timing_events=False):
        """``timing_events`` makes each CopyHandle.event a timing event, so a
        caller can measure the transfer on the copy stream (benchmarks)."""
        self.closed = False
        self._host_buffers = []
        self.thread = None
        self.queue = queue.SimpleQueue()
        self.gpu_num_pages = gpu_num_pages
        self.l2_num_pages = l2_num_pages
        transport = transport or DEFAULT_TRANSPORT
        assert transport in TRANSPORTS, f"unknown transport {transport!r}; pick one of {sorted(TRANSPORTS)}"
        self.transport = transport
        self._transport_code = TRANSPORTS[transport]
        self.device = gpu_caches[0].device
        assert all(c.is_cuda and c.device == self.device for c in gpu_caches)
        self.host_caches = [self._alloc_pinned_mirror(cache, l2_num_pages) for cache in gpu_caches]
        gpu_views = make_dma_views(gpu_caches, gpu_num_pages)
        cpu_views = make_dma_views(self.host_caches, l2_num_pages)
        max_pages = max(gpu_num_pages, l2_num_pages)
        self.load_params = _TransferParams(
            cpu_views, gpu_views, torch.cuda.Stream(self.device), l2_num_pages, gpu_num_pages, max_pages
        )
        self.store_params = _TransferParams(
            gpu_views, cpu_views, torch.cuda.Stream(self.device), gpu_num_pages, l2_num_pages, max_pages
        )
        if self._transport_code == _lib.SWAP_BLIT:
            self.load_params.alloc_staging(self.device)
            self.store_params.alloc_staging(self.device)
        self.thread = threading.Thread(
            target=self._copy_loop, args=(self.queue, self.device, self._transport_code, timing_events), daemon=True
        )
        self.thread.start()

    def __del__(self):
        self.close()

    def _alloc_pinned_mirror(self, cache, num_pages):
        """Host tensor shaped like ``cache`` but ``num_pages`` deep, pinned and
        mapped into the GPU's address space."""
        shape = list(cache.shape)
        shape[1] = num_pages
        nbytes = int(np.prod(shape, dtype=np.int64)) * cache.element_size()
        buf = _HostBuffer(max(nbytes, 1))
        self._host_buffers.append(buf)
        return buf.tensor(cache.dtype, tuple(shape))

    # -- submission ---------------------------------------------------------- #

    def store(self, gpu_page_idxs, l2_page_idxs):
        """D2H, ordered after the KV writes already queued on the current stream."""
        compute_done = torch.cuda.Event()
        compute_done.record(torch.cuda.current_stream(self.device))
        return self._submit(gpu_page_idxs, l2_page_idxs, is_store=True, wait_event=compute_done)

    def count_runs(self, src_ids, dst_ids):
        """Runs one transfer of these page pairs would make (as CopyHandle.num_runs)."""
        if not len(src_ids):
            return 0
        return len(self._coalesce(np.asarray(src_ids), np.asarray(dst_ids))[0])

    def load(self, l2_page_idxs, gpu_page_idxs):
        """H2D.  The caller must not read the GPU pages until the handle is waited on."""
        compute_done = torch.cuda.Event()
        compute_done.record(torch.cuda.current_stream(self.device))
        return self._submit(l2_page_idxs, gpu_page_idxs, is_store=False, wait_event=compute_done)

    def calibrate(self, num_pages=512):
        """Per-direction ``{desc_rate, bw}``, solving ``t = descriptors/desc_rate + bytes/bw``
        from a coalesced and a scattered transfer (copy_engine.py:286-333).
        Overwrites the first ``num_pages`` pages of both tiers."""
        n = min(num_pages, self.gpu_num_pages, self.l2_num_pages)
        fwd = list(range(n))
        rev = list(reversed(fwd))
        model = {}
        for direction, submit in (("store", self.store), ("load", self.load)):
            params = self.store_params if direction == "store" else self.load_params
            samples = {}
            for tag, dst in (("coalesced", fwd), ("scattered", rev)):
                for _ in range(2):  # the first pass pays warmup
                    start = time.perf_counter()
                    handle = submit(fwd, dst)
                    handle.wait()
                    elapsed = time.perf_counter() - start
                samples[tag] = (
                    handle.num_runs * params.num_tensors,
                    handle.num_pages * int(params.bpb.sum()),
                    elapsed,
                )
            (d_lo, nbytes, t_lo), (d_hi, _, t_hi) = samples["coalesced"], samples["scattered"]
            t_desc = min(max((t_hi - t_lo) / max(1, d_hi - d_lo), 1e-9), 1.0)
            link_s = max(t_lo - d_lo * t_desc, 1e-9)
            model[direction] = {"desc_rate": int(1 / t_desc), "bw": int(nbytes / link_s)}
        return model

    def close(self):
        if getattr(self, "closed", True):
            return
        self.closed = True
        if getattr(self, "thread", None) is not None:
            self.queue.put(None)
            self.thread.join(timeout=30.0)
        # Free pinned memory only once nothing in flight can touch it.
        for name in ("load_params", "store_params"):
            params = getattr(self, name, None)
            if params is not None:
                params.stream.synchronize()
                params.free()
        self.host_caches = []
        for buf in getattr(self, "_host_buffers", []):
            buf.free()
        self._host_buffers = []

    def _submit(self, src_ids, dst_ids, is_store, wait_event=None):
        assert not self.closed, "CopyEngine is closed"
        params = self.store_params if is_store else self.load_params
        if not len(src_ids):
            return CopyHandle(pending=False)
        src = np.array(src_ids, dtype=np.uint64)
        dst = np.array(dst_ids, dtype=np.uint64)
        assert src.shape == dst.shape, "source and destination page lists differ in length"
        self._check_range(src, dst, params.src_limit, params.dst_limit, is_store)
        if self._transport_code == _lib.SWAP_BLIT:
            assert len(src) <= params.max_pages, f"{len(src)} pages exceed one transfer's staging ({params.max_pages})"
        runs = self._coalesce(src, dst)
        handle = CopyHandle()
        handle.num_runs = len(runs[0])
        handle.num_pages = len(src_ids)
        self.queue.put((runs, wait_event, handle, params))
        # Hand the GIL to the copy thread so that it enqueues the transfer now: a
        # caller that goes on with a long Python loop (the ledger walking a
        # prompt) would otherwise hold it for up to the interpreter's 5 ms switch
        # interval per piece.  sleep(0) returns before the thread has woken.
        time.sleep(GIL_HANDOFF_S)
        return handle

    # -- copy thread --------------------------------------------------------- #

    @staticmethod
    def _check_range(src, dst, src_limit, dst_limit, is_store):
        """Raise before anything is enqueued for an index no pool owns
        (copy_engine.py:373-385)."""
        for ids, limit, side in ((src, src_limit, "src"), (dst, dst_limit, "dst")):
            if len(ids) and int(ids.max()) >= limit:
                bad = np.flatnonzero(ids >= limit)
                tier = ("gpu", "l2") if (side == "src") == is_store else ("l2", "gpu")
                raise AssertionError(
                    f"L2 {'store' if is_store else 'load'} {side} page index out of "
                    f"range for the {tier[0]} tier: "
                    f"{[int(ids[i]) for i in bad[:8]]} >= {limit} "
                    f"({len(bad)} of {len(ids)} pages bad)"
                )

    @classmethod
    def _copy_loop(cls, q, device, transport, timing=False):
        torch.cuda.set_device(device)
        while True:
            item = q.get()
            if item is None:
                return
            runs, wait_event, handle, params = item
            stream = params.stream
            try:
                with torch.cuda.stream(stream):
                    if wait_event is not None:
                        stream.wait_event(wait_event)
                    slot = params.next_staging() if transport == _lib.SWAP_BLIT else None
                    cls._copy_blocks(runs, params, transport, slot)
                    event = torch.cuda.Event(enable_timing=timing)
                    event.record(stream)
                    if slot is not None:
                        slot[1] = event
                handle.event = event
            except Exception as exc:  # deferred to CopyHandle.wait
                handle.error = exc

    @staticmethod
    def _coalesce(src_ids, dst_ids):
        """Merge page pairs that advance together on both tiers into runs
        (copy_engine.py:407-427): order by source (stable), split wherever the
        source or destination does not step by one.  Native (radix sort in
        libpipeswift_kv) because the caller waits for it.  Returns run starts
        on both sides and run lengths, in pages, as uint64 arrays."""
        src = np.ascontiguousarray(src_ids, dtype=np.int64)
        dst = np.ascontiguousarray(dst_ids, dtype=np.int64)
        n = len(src)
        rs = np.empty(n, dtype=np.int64)
        rd = np.empty(n, dtype=np.int64)
        rl = np.empty(n, dtype=np.int64)
        runs = lib().psk_coalesce_runs(src.ctypes.data_as(_i64p), dst.ctypes.data_as(_i64p), n,
                                       rs.ctypes.data_as(_i64p), rd.ctypes.data_as(_i64p), rl.ctypes.data_as(_i64p))
        if runs < 0:
            check(int(runs), "coalesce page runs")
        return rs[:runs].astype(np.uint64), rd[:runs].astype(np.uint64), rl[:runs].astype(np.uint64)

    @staticmethod
    def _copy_blocks(runs, params, transport, slot=None):
        """Enqueue the transfer of pre-coalesced page runs on params.stream."""
        src_start, dst_start, run_len = (np.ascontiguousarray(a, dtype=np.int64) for a in runs)
        if not len(run_len):
            return
        staging, staging_bytes = (slot[0].ptr, slot[0].nbytes) if slot is not None else (None, 0)
        desc = params.desc_dev
        desc_ptr, desc_bytes = (desc.data_ptr(), desc.numel()) if (slot is not None and desc is not None) else (None, 0)
        status = lib().psk_swap_blocks(
            transport,
            params.src_bases.ctypes.data_as(_u64p),
            params.dst_bases.ctypes.data_as(_u64p),
            params.bpb.ctypes.data_as(_u64p),
            params.num_tensors,
            src_start.ctypes.data_as(_i64p),
            dst_start.ctypes.data_as(_i64p),
            run_len.ctypes.data_as(_i64p),
            len(run_len),
            params.src_limit,
            params.dst_limit,
            staging,
            staging_bytes,
            desc_ptr,
            desc_bytes,
            params.stream_handle,
        )
        check(status, "L2 page transfer")
