"""DRAM L2 offload transport (swap_blocks) for MI355X.

Drop-in for pipeswift/utils/copy_engine.py: the same ``CopyEngine`` /
``CopyHandle`` / ``page_bytes`` / ``make_dma_views`` surface that
BlockManager calls (block_manager.py:190-209, 288, 462, 534), with the transfer
itself in ``psk_swap_blocks`` of libpipeswift_kv.so instead of a ctypes binding
of cuMemcpyBatchAsync.

The contract kept from the reference:
  * one pinned host mirror per GPU cache tensor, shaped like the cache but
    ``l2_num_pages`` deep, so page p of a layer spans the same byte range of
    that layer on both tiers;
  * runs of pages that advance together on both tiers are coalesced on the
    calling thread, so ``CopyHandle.num_runs`` (what the caller prices the
    retire deadline from) is known when ``store``/``load`` returns;
  * a transfer starts after the work already queued on the caller's stream,
    runs on a dedicated stream per direction and signals an event on it;
  * page indices are validated before anything is enqueued;
  * ``calibrate`` returns the ``t = descriptors/desc_rate + bytes/bw`` model
    with integer rates per direction.

The design underneath:
  * the per-(tensor, layer) byte geometry of each direction is computed once
    from the cache tensors' strides (``_Geometry``), as numpy arrays that go to
    the library as they are;
  * the mirror is hipHostMalloc'd (mapped, portable) by the library instead of
    taken from torch's caching pinned allocator, which would round a multi-GiB
    mirror up to the next power of two;
  * two transports: ``"blit"`` (default) moves every (view, page) unit of a
    transfer in ONE kernel that reads/writes the mapped host mirror directly,
    so the cost per descriptor that dominates the reference
    (copy_engine.py:15-36) disappears; ``"memcpy"`` issues one hipMemcpyAsync
    per (view, run) on the SDMA engines (the batched-descriptor call the
    reference uses has a HIP counterpart this GPU's runtime does not export);
  * one ``_Submitter`` thread owns every runtime call of the transfers, so
    the scheduler thread never blocks in the runtime; both copy streams keep
    the default priority.
"""

from __future__ import annotations

import ctypes
import math
import os
import queue
import threading
import time
import weakref
from collections import OrderedDict

import numpy as np
import torch

from . import _lib
from ._lib import check, lib

TRANSPORTS = {"memcpy": _lib.SWAP_MEMCPY, "blit": _lib.SWAP_BLIT}
DEFAULT_TRANSPORT = os.environ.get("PIPESWIFT_AMD_SWAP_TRANSPORT", "blit")
# Pinned page-table staging buffers per direction (blit transport): a buffer is
# reused only after the transfer that last read it has landed.
_STAGING_SLOTS = 4
# How long a submitter sleeps after queuing a transfer, so that the copy thread
# takes the GIL and enqueues it (CopyEngine._submit).
GIL_HANDOFF_S = 1e-4

_i64p = ctypes.POINTER(ctypes.c_int64)
_u64p = ctypes.POINTER(ctypes.c_uint64)


# --------------------------------------------------------------------------- #
# cache tensor layout (copy_engine.py:121-142)
# --------------------------------------------------------------------------- #


def page_bytes(caches):
    """Bytes one page occupies across every layer of every cache tensor (a
    cache is [layers, pages, ...])."""
    total = 0
    for cache in caches:
        per_layer = math.prod(cache.shape[2:]) * cache.element_size()
        total += cache.shape[0] * per_layer
    return total


def make_dma_views(caches, num_pages):
    """``{"<tensor>.<layer>": int8 [num_pages, bytes per page]}`` over every
    layer of every cache tensor.  The tensors must be contiguous, so a run of
    consecutive pages of one layer is one byte range."""
    out = OrderedDict()
    for ci, cache in enumerate(caches):
        if cache.shape[1] != num_pages or not cache.is_contiguous():
            raise AssertionError(f"cache {ci}: need a contiguous [layers, {num_pages}, ...] tensor, "
                                 f"got shape {tuple(cache.shape)}")
        flat = cache.view(cache.shape[0], num_pages, -1)
        for li in range(cache.shape[0]):
            out[f"{ci}.{li}"] = flat[li].view(torch.int8)
    return out


class _Geometry:
    """Byte geometry of one direction: for every (cache tensor, layer) view, the
    source and destination address of page 0 and the bytes per page, read from
    the tensors' strides (contiguous [layers, pages, ...] on both sides)."""

    def __init__(self, src_caches, dst_caches):
        src_b, dst_b, bpp = [], [], []
        for src, dst in zip(src_caches, dst_caches):
            if not (src.is_contiguous() and dst.is_contiguous()) or src.shape[0] != dst.shape[0] \
                    or src.shape[2:] != dst.shape[2:] or src.dtype != dst.dtype:
                raise AssertionError("mirror and cache tensors must be contiguous with matching page shapes")
            es = src.element_size()
            layers = np.arange(src.shape[0], dtype=np.uint64)
            src_b.append(np.uint64(src.data_ptr()) + layers * np.uint64(src.stride(0) * es))
            dst_b.append(np.uint64(dst.data_ptr()) + layers * np.uint64(dst.stride(0) * es))
            bpp.append(np.full(src.shape[0], src.stride(1) * es, dtype=np.uint64))
        self.src_bases = np.ascontiguousarray(np.concatenate(src_b))
        self.dst_bases = np.ascontiguousarray(np.concatenate(dst_b))
        self.bpb = np.ascontiguousarray(np.concatenate(bpp))
        self.num_tensors = len(self.bpb)


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
# page validation and coalescing
# --------------------------------------------------------------------------- #


def validate_pages(ids, limit, tier, what):
    """AssertionError naming the offending ids when any of ``ids`` is not a page
    of a ``limit``-page ``tier``; nothing is enqueued for such a transfer
    (copy_engine.py:373-385 checks the same before the driver call)."""
    ids = np.asarray(ids, dtype=np.int64)
    if not len(ids) or (int(ids.min()) >= 0 and int(ids.max()) < limit):
        return
    bad = ids[(ids < 0) | (ids >= limit)]
    shown = ", ".join(str(int(x)) for x in bad[:8]) + (", ..." if len(bad) > 8 else "")
    raise AssertionError(f"{what}: {len(bad)} of {len(ids)} page ids are not pages of the {tier} tier "
                         f"(it has {limit}): {shown}")


def coalesce_runs(src_ids, dst_ids):
    """Page pairs merged into runs that advance together on both tiers
    (copy_engine.py:407-427): pairs ordered by source (stable), cut wherever
    the source or the destination does not step by one.  The native radix
    sort in libpipeswift_kv does it, since the submitting caller waits.
    Returns (source starts, destination starts, lengths) as uint64 arrays."""
    src = np.ascontiguousarray(src_ids, dtype=np.int64)
    dst = np.ascontiguousarray(dst_ids, dtype=np.int64)
    n = len(src)
    out = np.empty((3, n), dtype=np.int64)
    runs = lib().psk_coalesce_runs(src.ctypes.data_as(_i64p), dst.ctypes.data_as(_i64p), n,
                                   out[0].ctypes.data_as(_i64p), out[1].ctypes.data_as(_i64p),
                                   out[2].ctypes.data_as(_i64p))
    if runs < 0:
        check(int(runs), "coalesce page runs")
    starts_s, starts_d, lengths = out[:, :runs].astype(np.uint64)
    return starts_s, starts_d, lengths


# --------------------------------------------------------------------------- #
# handles
# --------------------------------------------------------------------------- #


class CopyHandle:
    """One submitted transfer (copy_engine.py:150-177): ``event`` is recorded
    on the copy stream once the submitter has enqueued it; ``num_runs`` and
    ``num_pages`` are set before ``store``/``load`` returns."""

    def __init__(self, pending=True):
        self.event = None
        self.pending = pending  # False for an empty transfer, which never gets an event
        self.error = None
        self.num_runs = 0
        self.num_pages = 0

    def wait(self):
        """Block until the transfer has landed.  The submitter needs the GIL to
        enqueue it, so the wait for its event sleeps instead of spinning."""
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


# --------------------------------------------------------------------------- #
# one direction of the transport
# --------------------------------------------------------------------------- #


class _Lane:
    """One direction (store: GPU -> host, load: host -> GPU): its geometry, its
    copy stream, the page-count limits of both ends, and for the blit transport
    a ring of pinned page-table staging buffers plus the device buffer the
    table is copied into before each blit."""

    def __init__(self, name, geometry, stream, src_tier, dst_tier):
        self.name = name
        self.geometry = geometry
        self.num_tensors = geometry.num_tensors
        self.stream = stream
        self.src_tier, self.src_limit = src_tier
        self.dst_tier, self.dst_limit = dst_tier
        self.max_pages = max(self.src_limit, self.dst_limit)
        self._ring = []  # [host buffer, event of the last transfer that read it]
        self._next = 0
        self._desc = None

    def enable_staging(self, device):
        nbytes = int(lib().psk_swap_staging_bytes(self.num_tensors, self.max_pages))
        self._ring = [[_HostBuffer(nbytes), None] for _ in range(_STAGING_SLOTS)]
        self._desc = torch.empty(nbytes, dtype=torch.uint8, device=device)

    def check(self, src, dst):
        what = f"L2 {self.name}"
        validate_pages(src, self.src_limit, self.src_tier, f"{what} source")
        validate_pages(dst, self.dst_limit, self.dst_tier, f"{what} destination")
        if self._ring and len(src) > self.max_pages:
            raise AssertionError(f"{what}: {len(src)} pages exceed one transfer's staging ({self.max_pages})")

    def enqueue(self, runs, transport, timing):
        """Enqueue one transfer of coalesced runs on this lane's stream (called
        on the submitter thread, inside ``torch.cuda.stream(self.stream)``);
        returns the event recorded after it."""
        slot = None
        if self._ring:
            slot = self._ring[self._next]
            self._next = (self._next + 1) % len(self._ring)
            if slot[1] is not None:
                slot[1].synchronize()  # the transfer that last read this table has landed
        src_start, dst_start, run_len = (np.ascontiguousarray(a, dtype=np.int64) for a in runs)
        g = self.geometry
        if len(run_len):
            status = lib().psk_swap_blocks(
                transport, g.src_bases.ctypes.data_as(_u64p), g.dst_bases.ctypes.data_as(_u64p),
                g.bpb.ctypes.data_as(_u64p), g.num_tensors,
                src_start.ctypes.data_as(_i64p), dst_start.ctypes.data_as(_i64p), run_len.ctypes.data_as(_i64p),
                len(run_len), self.src_limit, self.dst_limit,
                slot[0].ptr if slot else None, slot[0].nbytes if slot else 0,
                self._desc.data_ptr() if slot else None, self._desc.numel() if slot else 0,
                self.stream.cuda_stream)
            check(status, "L2 page transfer")
        event = torch.cuda.Event(enable_timing=timing)
        event.record(self.stream)
        if slot is not None:
            slot[1] = event
        return event

    def release(self):
        """Drain the stream, then free the staging buffers."""
        self.stream.synchronize()
        for buf, _ in self._ring:
            buf.free()
        self._ring = []
        self._desc = None


class _Job:
    __slots__ = ("lane", "runs", "after", "handle")

    def __init__(self, lane, runs, after, handle):
        self.lane, self.runs, self.after, self.handle = lane, runs, after, handle


class _Submitter(threading.Thread):
    """The daemon thread that makes every runtime call of the transfers: it
    takes jobs in order, makes the lane's stream wait for the caller's event,
    enqueues the transfer and hands the recorded event to the job's handle.  A
    failure is parked on the handle and raised by its ``wait``."""

    def __init__(self, device, transport, timing):
        super().__init__(name="pipeswift-amd-l2-copy", daemon=True)
        self.jobs = queue.SimpleQueue()
        self._device = device
        self._transport = transport
        self._timing = timing

    def run(self):
        torch.cuda.set_device(self._device)
        for job in iter(self.jobs.get, None):
            try:
                with torch.cuda.stream(job.lane.stream):
                    if job.after is not None:
                        job.lane.stream.wait_event(job.after)
                    job.handle.event = job.lane.enqueue(job.runs, self._transport, self._timing)
            except Exception as exc:  # deferred to CopyHandle.wait
                job.handle.error = exc

    def stop(self, timeout=30.0):
        self.jobs.put(None)
        self.join(timeout=timeout)


def _shutdown(submitter, lanes, host_buffers):
    """Stop the submitter, drain both lanes, then free the pinned memory (only
    once nothing in flight can touch it).  Runs once: from ``close`` or when
    the engine is collected."""
    if submitter is not None and submitter.is_alive():
        submitter.stop()
    for lane in lanes:
        lane.release()
    for buf in host_buffers:
        buf.free()
    host_buffers.clear()


# --------------------------------------------------------------------------- #
# the engine
# --------------------------------------------------------------------------- #


class CopyEngine:
    """Pinned host mirror of the KV cache plus the page mover between tiers.

    ``store``/``load`` validate and coalesce on the calling thread, queue the
    transfer for the submitter thread, and return a CopyHandle at once; the
    transfers run on one dedicated stream per direction, overlapping compute.
    """

    def __init__(self, gpu_caches, gpu_num_pages, l2_num_pages, transport=None, timing_events=False):
        """``timing_events`` makes each CopyHandle.event a timing event, so a
        caller can measure the transfer on the copy stream (benchmarks)."""
        transport = transport or DEFAULT_TRANSPORT
        if transport not in TRANSPORTS:
            raise AssertionError(f"unknown transport {transport!r}; pick one of {sorted(TRANSPORTS)}")
        self.device = gpu_caches[0].device
        if not all(c.is_cuda and c.device == self.device for c in gpu_caches):
            raise AssertionError("every cache tensor must live on the same GPU")
        self.transport = transport
        self.gpu_num_pages = gpu_num_pages
        self.l2_num_pages = l2_num_pages
        self.closed = False
        self._buffers = []
        self.host_caches = []
        for cache in gpu_caches:
            if cache.shape[1] != gpu_num_pages:
                raise AssertionError(f"cache pages {cache.shape[1]} != gpu_num_pages {gpu_num_pages}")
            shape = (cache.shape[0], l2_num_pages) + tuple(cache.shape[2:])
            buf = _HostBuffer(max(1, math.prod(shape) * cache.element_size()))
            self._buffers.append(buf)
            self.host_caches.append(buf.tensor(cache.dtype, shape))
        gpu_end, l2_end = ("gpu", gpu_num_pages), ("l2", l2_num_pages)
        self.store_params = _Lane("store", _Geometry(gpu_caches, self.host_caches),
                                  torch.cuda.Stream(self.device), gpu_end, l2_end)
        self.load_params = _Lane("load", _Geometry(self.host_caches, gpu_caches),
                                 torch.cuda.Stream(self.device), l2_end, gpu_end)
        lanes = (self.store_params, self.load_params)
        code = TRANSPORTS[transport]
        if code == _lib.SWAP_BLIT:
            for lane in lanes:
                lane.enable_staging(self.device)
        self._submitter = _Submitter(self.device, code, timing_events)
        self._submitter.start()
        self._finalizer = weakref.finalize(self, _shutdown, self._submitter, lanes, self._buffers)

    # -- submission ---------------------------------------------------------- #

    def store(self, gpu_page_idxs, l2_page_idxs):
        """D2H, ordered after the KV writes already queued on the current stream."""
        return self._submit(self.store_params, gpu_page_idxs, l2_page_idxs)

    def load(self, l2_page_idxs, gpu_page_idxs):
        """H2D.  The caller must not read the GPU pages until the handle is waited on."""
        return self._submit(self.load_params, l2_page_idxs, gpu_page_idxs)

    def count_runs(self, src_ids, dst_ids):
        """Runs one transfer of these page pairs would make (as CopyHandle.num_runs)."""
        return len(coalesce_runs(src_ids, dst_ids)[2]) if len(src_ids) else 0

    def _submit(self, lane, src_ids, dst_ids):
        if self.closed:
            raise AssertionError("CopyEngine is closed")
        if not len(src_ids):
            return CopyHandle(pending=False)
        src = np.asarray(src_ids, dtype=np.int64)
        dst = np.asarray(dst_ids, dtype=np.int64)
        if src.shape != dst.shape:
            raise AssertionError(f"L2 {lane.name}: {len(src)} source pages but {len(dst)} destination pages")
        lane.check(src, dst)
        runs = coalesce_runs(src, dst)
        handle = CopyHandle()
        handle.num_runs, handle.num_pages = len(runs[2]), len(src)
        after = torch.cuda.Event()
        after.record(torch.cuda.current_stream(self.device))
        self._submitter.jobs.put(_Job(lane, runs, after, handle))
        # Hand the GIL to the submitter so that it enqueues the transfer now: a
        # caller going on with a long Python loop (the ledger walking a prompt)
        # would otherwise hold it for up to the interpreter's 5 ms switch
        # interval.  sleep(0) returns before the thread has woken.
        time.sleep(GIL_HANDOFF_S)
        return handle

    # -- cost model ---------------------------------------------------------- #

    def calibrate(self, num_pages=512):
        """Per-direction ``{desc_rate, bw}`` (integers) of the model
        ``seconds = descriptors / desc_rate + bytes / bw`` (copy_engine.py:286-333).

        Two transfers of the same n pages per direction: in order (few runs)
        and reversed on the destination (one run per page).  Each is timed from
        submission until its handle's wait returns (what a retire deadline has
        to cover), best of three after a warmup; the difference of the two
        times over the difference of their descriptor counts is the cost of a
        descriptor, and what the ordered transfer spent beyond its descriptors
        is the link time of its bytes.  Overwrites the first n pages of both
        tiers."""
        n = min(num_pages, self.gpu_num_pages, self.l2_num_pages)
        ids = np.arange(n, dtype=np.int64)
        model = {}
        for lane in (self.store_params, self.load_params):
            measured = []
            for dst in (ids, ids[::-1].copy()):
                self._time_transfer(lane, ids, dst)  # warmup
                seconds = min(self._time_transfer(lane, ids, dst) for _ in range(3))
                measured.append((self.count_runs(ids, dst) * lane.num_tensors, seconds))
            (d_in_order, t_in_order), (d_scattered, t_scattered) = measured
            per_desc = (t_scattered - t_in_order) / max(1, d_scattered - d_in_order)
            per_desc = min(max(per_desc, 1e-9), 1.0)  # scattering never speeds a transfer up
            link = max(t_in_order - d_in_order * per_desc, 1e-9)
            nbytes = n * int(lane.geometry.bpb.sum())
            model[lane.name] = {"desc_rate": int(1.0 / per_desc), "bw": int(nbytes / link)}
        return model

    def _time_transfer(self, lane, src, dst):
        """Wall seconds from submitting one transfer until it has landed."""
        torch.cuda.synchronize(self.device)
        t0 = time.perf_counter()
        self._submit(lane, src, dst).wait()
        return time.perf_counter() - t0

    # -- shutdown ------------------------------------------------------------ #

    def close(self):
        """Stop the submitter, drain both copy streams, free the pinned mirror.
        Idempotent; also runs when the engine is garbage-collected."""
        if self.closed:
            return
        self.closed = True
        self._finalizer()
        self.host_caches = []
