"""Page ledger of the paged KV cache: which HBM pages each sequence owns, the
prefix cache over them, and the pinned-host L2 tier with its deadline-priced
transfers.

Drop-in for pipeswift/engine/block_manager.py -- ``L2PagePool`` (:22-121) and
``BlockManager`` (:124-885) -- with the same public names, arguments and
behaviour (page ids, eviction order, counters, retire steps).  The structure is
this module's own: both tiers share one refcounted ``_PagePool``;
``BlockManager`` is the HBM tier and owns an ``_L2Tier`` that holds everything
behind it (pool, copy engine, agreed cost model, the ``_LinkClock`` that prices
deadlines, staged requests, and one FIFO of in-flight ``_Transfer`` records per
direction), exposing its state under the reference's attribute names.  The
bytes move through the HIP ``CopyEngine`` (a blit kernel over mapped pinned
memory, one launch per batch) and the prefix-chained page keys come from one
native call per prompt (``psk_page_hash_chain``) instead of one xxhash object
per page.

Two deliberate departures, both confined to states in which the reference
hands one page to two owners:

* ``allocate_prefill`` takes its references on the matched L1 prefix before it
  allocates restore targets and fresh pages.  The reference allocates first
  (block_manager.py:741-767), so when the free queue is empty the LRU eviction
  can recycle a matched prefix page as a restore target: the page then appears
  twice in one page table and the restore overwrites the prefix.
* A staged restore pins its pages (the L2 source and the GPU target) when it is
  staged, not when it is flushed (:509-548).  Between the two, a store batch can
  evict the L2 source, and a sequence released before the flush returns its
  target to the free queue while the flush still writes it.

In every other state, page ids, eviction order, counters and retire steps are
the reference's, call for call.
"""

from __future__ import annotations

import ctypes
import functools
import gc
import itertools
import math
import warnings
import weakref
from array import array
from collections import OrderedDict, deque
from typing import Dict, List

import numpy as np
import torch
import torch.distributed as dist

from . import copy_engine
from ._lib import check, lib

DEFAULT_L2_STEP_MS = 10.0  # block_manager.py:15
# Decode headroom (tokens) every sequence holding pages must keep before the
# pool is spent on a waiting one (block_manager.py:16-19).
DECODE_RESERVE_TOKENS = 512
# Pages per submitted piece of one L2 store batch (_schedule_l2_store_batch).
L2_STORE_CHUNK = 1024
# Pages per restore piece submitted while allocate_prefill walks a prompt.
L2_LOAD_CHUNK = 1024
# The first piece of a batch or prompt is this many pages (at most the chunk)
# and each later one twice the one before, up to the chunk: the link starts
# after the host has walked 128 pages (~0.2 ms) instead of 1024 (~1.4 ms).
L2_FIRST_PIECE = 128


def _collector_paused(fn):
    """Run a ledger walk with Python's cyclic garbage collector held off, its
    previous state restored afterwards (on an error too).  A walk over a long
    prompt allocates a few containers per page (page keys, restore records);
    with the collector on, their allocations trigger collections that rescan
    them and the rest of the heap every few hundred pages, which made a
    16000-page store or restore walk about 3x slower on the host (114 / 122 ms
    against 37 / 41 ms).  Reference counting frees objects as usual meanwhile;
    only the detection of reference cycles waits for the walk to end."""

    @functools.wraps(fn)
    def run(*args, **kwargs):
        if not gc.isenabled():
            return fn(*args, **kwargs)
        gc.disable()
        try:
            return fn(*args, **kwargs)
        finally:
            gc.enable()

    return run


class _StagedLoads(list):
    """A sequence's staged restores (one dict per page, as the reference stages
    them), plus the copies already submitted for them and whether their pages
    are pinned; the flush joins those copies into its transfers."""

    __slots__ = ("handles", "pinned")

    def __init__(self):
        super().__init__()
        self.handles = []
        self.pinned = False


# --------------------------------------------------------------------------- #
# prefix keys
# --------------------------------------------------------------------------- #


def _token_buffer(token_ids):
    """(address, element bytes, count, keepalive) of ``token_ids`` laid out the
    way ``np.array(token_ids).tobytes()`` lays it out (block_manager.py:226)."""
    if isinstance(token_ids, array):
        addr, n = token_ids.buffer_info()
        return addr, token_ids.itemsize, n, token_ids
    a = np.ascontiguousarray(np.asarray(token_ids))
    return a.ctypes.data, a.itemsize, a.size, a


def page_key(token_ids, prefix: int = -1) -> int:
    """XXH64 of ``le64(prefix)`` (omitted when prefix is -1) followed by the
    token bytes: ``BlockManager.compute_hash`` (block_manager.py:220-227)."""
    addr, itemsize, n, keep = _token_buffer(token_ids)
    out = ctypes.c_uint64()
    st = lib().psk_keyed_hash(addr if n else None, n * itemsize, 0 if prefix == -1 else prefix, int(prefix != -1),
                              ctypes.addressof(out))
    check(st, "page_key")
    del keep
    return out.value


def page_key_chain(token_ids, page_size: int) -> List[int]:
    """Prefix-chained keys of every full page of ``token_ids``: page 0 keyed by
    its tokens alone, page i by key i-1 and its tokens (block_manager.py:681-688)."""
    addr, itemsize, n, keep = _token_buffer(token_ids)
    pages = n // page_size
    if pages == 0:
        return []
    keys = np.empty(pages, dtype=np.uint64)
    got = lib().psk_page_hash_chain(addr, n, itemsize, page_size, 0, 0, keys.ctypes.data, pages)
    if got < 0:
        check(int(got), "page_key_chain")
    del keep
    return keys.tolist()


# --------------------------------------------------------------------------- #
# refcounted pool
# --------------------------------------------------------------------------- #


class _PagePool:
    """Refcounted pages with a prefix-key index, the discipline both tiers share
    (block_manager.py:22-121 for L2, :144-166, :327-400, :784-840 for L1).

    Every page is in exactly one state:
      held    ``ref_counts[p] > 0``;
      free    ref 0, no key, in the FIFO ``free_page_queue``;
      cached  ref 0, keyed, in ``cached_pages`` (ordered; the head is evicted first).
    ``hash2page_idx_list[h]`` lists the keyed pages of key ``h`` in the order they
    were keyed; a lookup returns the first whose tokens match.
    """

    def __init__(self, num_pages: int, first_page: int = 0):
        self.num_pages = num_pages
        self.ref_counts = array("i", bytes(4 * num_pages))  # plain ints: no numpy scalar per access
        self.free_page_queue = deque(range(first_page, num_pages))
        self.cached_pages = OrderedDict()
        self.hash2page_idx_list: Dict[int, List[int]] = {}
        self.page_idx2token_ids = {}
        self.page_idx2hash = [-1] * num_pages

    def _find(self, h, token_ids):
        if h == -1:
            return None
        for p in self.hash2page_idx_list.get(h, ()):
            if self.page_idx2token_ids[p] == token_ids:
                return p
        return None

    def _key_page(self, p, h, token_ids):
        self.page_idx2hash[p] = h
        self.page_idx2token_ids[p] = token_ids
        self.hash2page_idx_list.setdefault(h, []).append(p)

    def _unkey_page(self, p):
        assert self.ref_counts[p] == 0
        h = self.page_idx2hash[p]
        pages = self.hash2page_idx_list.get(h) if h != -1 else None
        if pages is not None:
            if p in pages:
                pages.remove(p)
            if not pages:
                del self.hash2page_idx_list[h]
        self.page_idx2hash[p] = -1
        self.page_idx2token_ids[p] = []

    def _hold(self, p):
        """One more reference; a cached page leaves the eviction queue."""
        if self.ref_counts[p] == 0 and p in self.cached_pages:
            del self.cached_pages[p]
        self.ref_counts[p] += 1

    def _drop(self, p):
        """One reference fewer; at zero a keyed page joins the eviction queue's
        tail and an unkeyed one the free queue's."""
        self.ref_counts[p] -= 1
        assert self.ref_counts[p] >= 0
        if self.ref_counts[p] == 0:
            if self.page_idx2hash[p] == -1:
                self.free_page_queue.append(p)
            else:
                self.cached_pages[p] = None

    def _take_many(self, n):
        """``n`` pages with one reference each, the pages and order of ``n``
        calls of ``_take``; the caller has checked that the free and cached
        queues together hold at least ``n``."""
        free, rc = self.free_page_queue, self.ref_counts
        k = min(n, len(free))
        out = [free.popleft() for _ in range(k)]
        if k < n:
            # evict the cached queue's head n - k times, unkeying as _unkey_page does
            cached, p2h, p2t, h2l = self.cached_pages, self.page_idx2hash, self.page_idx2token_ids, self.hash2page_idx_list
            for _ in range(n - k):
                p = cached.popitem(last=False)[0]
                assert rc[p] == 0
                h = p2h[p]
                same = h2l.get(h) if h != -1 else None
                if same is not None:
                    if p in same:
                        same.remove(p)
                    if not same:
                        del h2l[h]
                p2h[p] = -1
                p2t[p] = []
                out.append(p)
        for p in out:
            assert rc[p] == 0
            rc[p] = 1
        return out

    def _take(self):
        """A page with one reference: the free queue's head, else the evicted
        (and unkeyed) head of the cached queue.  None when every page is held."""
        if self.free_page_queue:
            p = self.free_page_queue.popleft()
        elif self.cached_pages:
            p, _ = self.cached_pages.popitem(last=False)
            self._unkey_page(p)
        else:
            return None
        assert self.ref_counts[p] == 0
        self.ref_counts[p] = 1
        return p


class L2PagePool(_PagePool):
    """Host page ledger of the L2 tier (block_manager.py:22-121).  Besides the
    pool it counts the (key, tokens) pairs of stores that are staged or in
    flight, so a duplicate store is refused in O(1)."""

    def __init__(self, num_pages: int):
        super().__init__(num_pages)
        self._pending_store_keys = {}

    def lookup(self, h, token_ids):
        """The page holding this key and tokens, else None (:43-50)."""
        return self._find(h, token_ids)

    def has_page_or_pending(self, h, token_ids):
        """Resident, or already on its way (:52-58)."""
        if h == -1:
            return False
        if (h, tuple(token_ids)) in self._pending_store_keys:
            return True
        return self._find(h, token_ids) is not None

    def acquire_pending_key(self, key):
        self._pending_store_keys[key] = self._pending_store_keys.get(key, 0) + 1

    def release_pending_key(self, key):
        left = self._pending_store_keys.get(key, 0) - 1
        if left > 0:
            self._pending_store_keys[key] = left
        else:
            self._pending_store_keys.pop(key, None)

    def allocate_for_store(self):
        """A page to store into, evicting the LRU one if needed; None when all
        are pinned (:70-81)."""
        return self._take()

    def _reset_page(self, page_idx):
        self._unkey_page(page_idx)

    def retain_for_load(self, page_idx):
        """Pin a resident page for the duration of an H2D (:97-101)."""
        self._hold(page_idx)

    def release_from_load(self, page_idx):
        self._drop(page_idx)

    def finish_store(self, page_idx, h, token_ids):
        """Drop the store's pin and make the page discoverable (:109-117)."""
        self.ref_counts[page_idx] -= 1
        assert self.ref_counts[page_idx] >= 0
        self._key_page(page_idx, h, token_ids)
        if self.ref_counts[page_idx] == 0:
            self.cached_pages[page_idx] = None

    def get_usage(self):
        return 1 - len(self.free_page_queue) / self.num_pages


# --------------------------------------------------------------------------- #
# the L2 tier: link clock, in-flight transfers, staged requests
# --------------------------------------------------------------------------- #


class _Transfer:
    """A batched copy between the tiers that is in flight, and the scheduler
    step by which it is due to have landed.  A store carries the pages it
    reads and writes and the (key, tokens) of each; a restore carries the
    (sequence, staged loads) pairs it serves."""

    __slots__ = ("copy", "due_step", "gpu_page_idxs", "l2_page_idxs", "keys", "token_ids_list", "seq_loads")

    def __init__(self, copy, due_step, gpu_page_idxs=(), l2_page_idxs=(), keys=(), token_ids_list=(), seq_loads=()):
        self.copy = copy
        self.due_step = due_step
        self.gpu_page_idxs = gpu_page_idxs
        self.l2_page_idxs = l2_page_idxs
        self.keys = keys
        self.token_ids_list = token_ids_list
        self.seq_loads = seq_loads


class _LinkClock:
    """Per-direction water level of link-seconds the copy engine still owes.

    A direction drains serially, so a transfer lands after everything queued
    ahead of it: charging a transfer raises its direction's level (floored at
    the current step, since time the engine has had counts as drained) by
    ``runs * views / desc_rate + pages * page_bytes / bw`` and prices the due
    step as the level in steps, rounded up (block_manager.py:617-636).  Every
    input is agreed over ranks, so every rank predicts the same step."""

    def __init__(self, cost_model, views, page_bytes, step_ms):
        self.model = cost_model
        self.views = views
        self.page_bytes = page_bytes
        self.step_s = step_ms / 1000
        self.owed = {"store": 0.0, "load": 0.0}

    def seconds(self, direction, runs, pages):
        rates = self.model[direction]
        return runs * self.views / rates["desc_rate"] + pages * self.page_bytes / rates["bw"]

    def charge(self, direction, copy, now_step):
        level = max(self.owed[direction], now_step * self.step_s) + self.seconds(direction, copy.num_runs,
                                                                                   copy.num_pages)
        self.owed[direction] = level
        return int(math.ceil(level / self.step_s))

    def scattered_page_seconds(self):
        """One restored page priced fully scattered: a run per page per view
        (:646-655)."""
        return self.seconds("load", 1, 1)

    def restore_backlog_steps(self, now_step, extra_pages):
        """Steps until a restore of ``extra_pages`` more pages would land: the
        load level still ahead of the current step plus those pages (:657-672)."""
        ahead = max(self.owed["load"] - now_step * self.step_s, 0.0)
        return int(math.ceil((ahead + extra_pages * self.scattered_page_seconds()) / self.step_s))


def _step_sized_groups(staged, budget):
    """Consecutive (sequence, loads) entries cut into groups of at most
    ``budget`` pages, at whole sequences only; a sequence larger than the
    budget forms a group of its own (:550-567)."""
    group, room = [], budget
    for entry in staged:
        size = len(entry[1])
        if group and size > room:
            yield group
            group, room = [], budget
        group.append(entry)
        room -= size
    if group:
        yield group


def _due_prefix(transfers, now_step):
    """How many transfers at the head of ``transfers`` are due at ``now_step``
    (due steps never decrease along a direction's queue)."""
    return sum(1 for _ in itertools.takewhile(lambda t: t.due_step <= now_step, transfers))


class _L2Tier:
    """The pinned-host tier behind the HBM pool: its page pool and copy engine,
    the agreed cost model and geometry, the link clock, the stores and
    restores staged for the step's flush, and the transfers in flight (one
    FIFO per direction).  The BlockManager owning it keeps the HBM side."""

    def __init__(self, owner, l2_cache_gb, step_ms):
        # One tensor per layer stack where the layout allows it, so that a page
        # of a layer is one contiguous run (:176-189).
        if owner.mla_cache_tensor is not None:
            caches = [owner.mla_cache_tensor]
        elif owner.kv_cache_tensor is not None:
            caches = [owner.kv_cache_tensor]
        else:
            caches = list(owner.kv_cache)
        agree = owner._min_across_workers
        self.num_pages = self._agreed_num_pages(owner.num_pages, l2_cache_gb, caches, agree)
        self.engine = copy_engine.CopyEngine(caches, owner.num_pages, self.num_pages)
        self.pool = L2PagePool(self.num_pages)
        measured = self.engine.calibrate()
        self.cost_model = {d: {term: max(1, agree(int(v))) for term, v in rates.items()}
                           for d, rates in measured.items()}
        self.page_bytes = max(1, agree(copy_engine.page_bytes(caches)))
        self.views = max(1, agree(self.engine.load_params.num_tensors))
        self.clock = _LinkClock(self.cost_model, self.views, self.page_bytes, step_ms)
        self.now = 0  # the retire clock: the scheduler step
        self.staged_stores = []  # (gpu page, (key, tuple(tokens)), tokens)
        self.staged_loads = []  # (sequence, _StagedLoads)
        self.stores = deque()  # _Transfer, in submission order
        self.loads = deque()
        # The engine is closed when the tier is collected, also without close().
        weakref.finalize(self, self.engine.close)

    @staticmethod
    def _agreed_num_pages(gpu_pages, l2_cache_gb, caches, agree):
        """Pages of the byte budget, the minimum over ranks (:233-267)."""
        pb = copy_engine.page_bytes(caches)
        budget = int(l2_cache_gb * 1024**3 + 0.5)
        mine = budget // pb
        if mine <= 0:
            raise ValueError(f"L2 cache byte budget is too small: per_rank_budget={budget} bytes, page_bytes={pb}")
        pages = agree(mine)
        if pages < mine:
            warnings.warn(f"L2 cache pages lowered to the minimum over ranks: local={mine}, agreed={pages}",
                          RuntimeWarning)
        if pages < gpu_pages:
            warnings.warn("L2 cache holds fewer pages than the GPU pool, so only part of what L1 evicts fits; "
                          f"num_pages={gpu_pages}, l2_pages={pages}, per_rank_budget={budget} bytes, "
                          f"page_bytes={pb}", RuntimeWarning)
        return pages

    # -- stores (GPU -> host) ------------------------------------------------ #

    def stage_store(self, page_idx, h, token_ids):
        """Queue a store of a page decode just completed, for the step's flush,
        unless its (key, tokens) is in L2 or already on its way (:393-404)."""
        key = (h, tuple(token_ids))
        if key in self.pool._pending_store_keys or self.pool._find(h, token_ids) is not None:
            return False
        self.pool.acquire_pending_key(key)
        self.staged_stores.append((page_idx, key, token_ids))
        return True

    def submit_stores(self, owner, stores):
        """One logical D2H transfer of every (page, key, tokens) of ``stores``
        not resident or on its way, stopping at the first one no L2 page can
        take (:433-474).  Each accepted page is pinned on both tiers and its
        key claimed at once, so a duplicate later in the batch is skipped.

        The transfer goes to the engine in pieces (L2_FIRST_PIECE pages,
        doubling up to L2_STORE_CHUNK) while the batch is still being walked,
        so the link starts on the first pages instead of after the whole
        batch's bookkeeping (about 12 ms for an 8192-page prompt); its deadline
        is priced from the whole batch's runs, as for a single submission.
        Returns the pages sent."""
        pending, find, take = self.pool._pending_store_keys, self.pool._find, self.pool.allocate_for_store
        hold = owner._hold
        src, dst, keys, toks, pieces = [], [], [], [], []
        sent, piece = 0, min(L2_FIRST_PIECE, L2_STORE_CHUNK)
        for page_idx, h, token_ids in stores:
            key = (h, tuple(token_ids))
            if h != -1 and (key in pending or find(h, token_ids) is not None):
                continue
            q = take()
            if q is None:
                break  # every L2 page is pinned by a transfer
            pending[key] = pending.get(key, 0) + 1
            hold(page_idx)
            src.append(page_idx)
            dst.append(q)
            keys.append(key)
            toks.append(token_ids)
            if len(src) - sent >= piece:
                pieces.append(self.engine.store(src[sent:], dst[sent:]))
                sent, piece = len(src), min(2 * piece, L2_STORE_CHUNK)
        if not src:
            return 0
        if sent < len(src):
            pieces.append(self.engine.store(src[sent:], dst[sent:]))
        copy = pieces[0] if len(pieces) == 1 else copy_engine.JoinedCopyHandle(
            pieces, self.engine.count_runs(src, dst), len(src))
        self.stores.append(_Transfer(copy, self.clock.charge("store", copy, self.now), gpu_page_idxs=src,
                                     l2_page_idxs=dst, keys=keys, token_ids_list=toks))
        owner.l2_store_cnt += len(src)
        return len(src)

    def retire_stores(self, owner, count):
        """Land the ``count`` oldest stores (completion is FIFO): their L2 pages
        become discoverable, their keys stop pending, and the GPU pages they
        read are released suffix first (:476-491)."""
        pool = self.pool
        for _ in range(count):
            t = self.stores.popleft()
            t.copy.wait()
            for q, key, token_ids in zip(t.l2_page_idxs, t.keys, t.token_ids_list):
                pool.finish_store(q, key[0], token_ids)
                pool.release_pending_key(key)
            for p in reversed(t.gpu_page_idxs):
                owner._drop(p)

    # -- restores (host -> GPU) ---------------------------------------------- #

    def pin_loads(self, owner, loads):
        """Pin both pages of each restore: the GPU target and the L2 source."""
        hold, hold2 = owner._hold, self.pool._hold
        for load in loads:
            hold(load["gpu_page_idx"])
            hold2(load["l2_page_idx"])

    def stage_loads(self, owner, seq, loads):
        """Queue a sequence's restores for the batched flush (:497-507).  Their
        pages are pinned now (or were, when their copies went out while the
        prompt was allocated), so nothing recycles them before the flush."""
        if not getattr(loads, "pinned", False):
            self.pin_loads(owner, loads)
        seq.l2_load_pending = True
        self.staged_loads.append((seq, loads))

    def flush_loads(self, owner):
        """Send the staged restores as transfers of about one scheduler step of
        fully scattered pages each, cut at whole sequences (:509-548).  Copies
        that went out while their prompt was allocated join their group's
        transfer as they are; the group's other pages go now.  Returns the
        pages restored."""
        staged, self.staged_loads = self.staged_loads, []
        budget = max(1, int(self.clock.step_s / self.clock.scattered_page_seconds()))
        total = 0
        for group in _step_sized_groups(staged, budget):
            handles, src, dst, late = [], [], [], []
            for _, loads in group:
                early = getattr(loads, "handles", None)
                handles.extend(early or ())
                for load in loads:
                    src.append(load["l2_page_idx"])
                    dst.append(load["gpu_page_idx"])
                    if not early:
                        late.append(load)
            if late:
                handles.append(self.engine.load([ld["l2_page_idx"] for ld in late],
                                                [ld["gpu_page_idx"] for ld in late]))
            copy = handles[0] if len(handles) == 1 else copy_engine.JoinedCopyHandle(
                handles, self.engine.count_runs(src, dst), len(dst))
            self.loads.append(_Transfer(copy, self.clock.charge("load", copy, self.now), seq_loads=group))
            total += len(dst)
        owner.l2_load_cnt += total
        return total

    def retire_loads(self, owner, count):
        """Land the ``count`` oldest restores: key their GPU pages, unpin both
        tiers (a GPU page reaches zero references only for a sequence released
        mid-restore; suffix first), and move each live sequence past its
        restored pages (:569-592)."""
        ps = owner.page_size
        for _ in range(count):
            t = self.loads.popleft()
            t.copy.wait()
            for seq, loads in t.seq_loads:
                live = seq.seq_id in owner.kv_page_table
                for load in loads:
                    owner._publish_gpu_page(load["gpu_page_idx"], load["hash"], load["token_ids"])
                    self.pool.release_from_load(load["l2_page_idx"])
                for load in reversed(loads):
                    owner._drop(load["gpu_page_idx"])
                if live:
                    seq.offset += len(loads) * ps
                seq.l2_load_pending = False

    # -- the step clock ------------------------------------------------------ #

    def advance(self, owner, step_idx):
        """Step ``step_idx`` has run: land every transfer due by the next one,
        stores before restores (:608-615)."""
        self.now = step_idx + 1
        self.retire_stores(owner, _due_prefix(self.stores, self.now))
        self.retire_loads(owner, _due_prefix(self.loads, self.now))


# --------------------------------------------------------------------------- #
# block manager
# --------------------------------------------------------------------------- #


class BlockManager(_PagePool):
    """L1 page pool with prefix caching, and the L2 tier behind it
    (block_manager.py:124-885).  Page 0 is never handed out (:152), so padded
    page-table entries (0) never alias a live page."""

    def __init__(
        self,
        num_pages,
        page_size,
        kv_cache,
        mla_cache_tensor,
        kv_cache_tensor=None,
        l2_cache_gb=0,
        l2_step_ms=DEFAULT_L2_STEP_MS,
    ):
        if l2_step_ms <= 0:
            raise ValueError(f"l2_step_ms must be positive, got {l2_step_ms}")
        super().__init__(num_pages, first_page=1)
        self.page_size = page_size
        self.kv_page_table: Dict[int, array] = {}
        self.kv_cache: List[torch.Tensor] = kv_cache
        self.mla_cache_tensor: torch.Tensor = mla_cache_tensor
        # The fused [L, P, 2, ps, H, D] allocation ``kv_cache`` is viewed from.
        self.kv_cache_tensor: torch.Tensor = kv_cache_tensor
        # Assumed scheduler step: converts predicted link-seconds into the step
        # count a retire deadline is expressed in.
        self.l2_step_ms = l2_step_ms
        # prefix-cache hits in L1, pages restored from L2, pages stored / restored
        self.hit_cnt = self.l2_hit_cnt = self.l2_store_cnt = self.l2_load_cnt = 0
        self.l2 = _L2Tier(self, l2_cache_gb, l2_step_ms) if l2_cache_gb > 0 else None

    # The L2 tier's state under the reference's attribute names.
    enable_l2_cache = property(lambda self: self.l2 is not None)
    l2_pool = property(lambda self: self.l2.pool if self.l2 else None)
    l2_copy_engine = property(lambda self: self.l2.engine if self.l2 else None)
    l2_cost_model = property(lambda self: self.l2.cost_model if self.l2 else None)
    l2_num_pages = property(lambda self: self.l2.num_pages if self.l2 else 0)
    l2_page_bytes = property(lambda self: self.l2.page_bytes if self.l2 else 0)
    l2_views = property(lambda self: self.l2.views if self.l2 else 0)
    l2_step = property(lambda self: self.l2.now if self.l2 else 0)
    pending_l2_stores = property(lambda self: self.l2.stores if self.l2 else ())
    pending_l2_loads = property(lambda self: self.l2.loads if self.l2 else ())
    _l2_pending_store_requests = property(lambda self: self.l2.staged_stores if self.l2 else [])
    _l2_pending_load_requests = property(lambda self: self.l2.staged_loads if self.l2 else [])
    _l2_owed_s = property(lambda self: self.l2.clock.owed if self.l2 else {"store": 0.0, "load": 0.0})

    @classmethod
    def compute_hash(cls, token_ids, prefix: int = -1):
        return page_key(token_ids, prefix)

    @staticmethod
    def _min_across_workers(value):
        """Minimum over every rank of an initialised process group, else
        ``value`` (mpu.py:31-47).  gloo reduces a host tensor."""
        if not dist.is_available() or not dist.is_initialized() or dist.get_world_size() == 1:
            return value
        device = "cuda" if dist.get_backend() == "nccl" else "cpu"
        t = torch.tensor([value], dtype=torch.int64, device=device)
        dist.all_reduce(t, op=dist.ReduceOp.MIN)
        return int(t.item())

    # -- L1 pool ------------------------------------------------------------ #

    def can_allocate(self, seq, reserve_tokens: int = 0):
        held = len(self.kv_page_table.get(seq.seq_id, ()))
        need = (len(seq.token_ids) + reserve_tokens + self.page_size - 1) // self.page_size
        return self.free_pages() >= max(0, need - held)

    def free_pages(self):
        """Pages the pool can hand out, evictable cached ones included."""
        return len(self.free_page_queue) + len(self.cached_pages)

    def decode_reserve_pages(self, num_seqs):
        """Pages for ``num_seqs`` sequences to decode DECODE_RESERVE_TOKENS more
        each, the partial last page included (:313-320)."""
        return num_seqs * ((DECODE_RESERVE_TOKENS + self.page_size - 1) // self.page_size)

    def can_allocate_overlap_schedule(self, seqs):
        need = 0
        for seq in seqs:
            held = len(self.kv_page_table.get(seq.seq_id, ()))
            need += max(0, (len(seq.token_ids) + self.page_size) // self.page_size - held)
        return self.free_pages() >= need

    def allocate_a_page(self):
        """Free page, else evicted cached page; an in-flight store pins the GPU
        pages it reads, so those are drained before giving up (:327-345)."""
        while not self.free_page_queue and not self.cached_pages and self.reclaim_l2_store_pages():
            pass
        p = self._take()
        if p is None:
            raise RuntimeError("Out of KV Pages!")
        return p

    def _lookup_cached_page(self, h, token_ids):
        return self._find(h, token_ids)

    def _publish_gpu_page(self, page_idx, h, token_ids):
        if self.page_idx2hash[page_idx] == -1:
            self._key_page(page_idx, h, token_ids)

    def reset_page(self, page_idx):
        self._unkey_page(page_idx)

    def update_page(self, page_idx, h, token_ids, from_decode=False):
        """Key a page this sequence alone holds; pages completed by decode are
        also staged for L2 (:814-832)."""
        assert h != -1 and self.page_idx2hash[page_idx] == -1 and self.ref_counts[page_idx] == 1
        self._key_page(page_idx, h, token_ids)
        if from_decode and self.l2 is not None:
            self.l2.stage_store(page_idx, h, token_ids)

    def get_usage(self):
        return 1 - (len(self.free_page_queue) + len(self.cached_pages)) / self.num_pages

    def get_l2_usage(self):
        return self.l2.pool.get_usage() if self.l2 else 0.0

    # -- L2 calls of the scheduler (block_manager.py:393-672) --------------- #

    def flush_l2_stores(self):
        """Send the staged stores whose page still carries the staged key (a
        page can be merged away or recycled in between); returns the pages
        sent."""
        if self.l2 is None or not self.l2.staged_stores:
            return 0
        staged, self.l2.staged_stores = self.l2.staged_stores, []
        live = []
        for page_idx, key, token_ids in staged:
            self.l2.pool.release_pending_key(key)
            if self.page_idx2hash[page_idx] == key[0]:
                live.append((page_idx, key[0], token_ids))
        return self.l2.submit_stores(self, live)

    @_collector_paused
    def schedule_l2_stores_for_confirmed_seq(self, seq):
        """Store the keyed pages of the sequence's confirmed tokens (:420-431)."""
        if self.l2 is None or seq.seq_id not in self.kv_page_table:
            return
        table = self.kv_page_table[seq.seq_id]
        confirmed = table[: min(len(seq.token_ids) // self.page_size, len(table))]
        key_of, tokens_of = self.page_idx2hash, self.page_idx2token_ids
        self.l2.submit_stores(self, [(p, key_of[p], tokens_of[p]) for p in confirmed if key_of[p] != -1])

    @_collector_paused
    def flush_l2_loads(self):
        """Send the staged restores (see _L2Tier.flush_loads); returns the pages."""
        if self.l2 is None or not self.l2.staged_loads:
            return 0
        return self.l2.flush_loads(self)

    def reclaim_l2_store_pages(self):
        """Land the oldest in-flight store ahead of its deadline, freeing the GPU
        pages it pins; True if there was one (:594-606)."""
        if self.l2 is None or not self.l2.stores:
            return False
        self.l2.retire_stores(self, 1)
        return True

    def poll_l2_events(self, step_idx):
        """Once per scheduler step: land every transfer whose deadline step has
        arrived."""
        if self.l2 is not None:
            self.l2.advance(self, step_idx)

    @property
    def l2_page_s(self):
        """Link-seconds of one restored page priced fully scattered."""
        return self.l2.clock.scattered_page_seconds()

    def l2_load_horizon_steps(self):
        """Steps until a restore staged now would be due: the load level still
        owed past the current step plus the staged, unflushed pages."""
        if self.l2 is None:
            return 0
        staged = sum(len(loads) for _, loads in self.l2.staged_loads)
        return self.l2.clock.restore_backlog_steps(self.l2.now, staged)

    # -- sequence-level allocation ----------------------------------------- #


    def _prompt_page_hashes(self, seq):
        """``[(key, page tokens)]`` for every page of the prompt, -1 for a
        partial last page, cached on the sequence by token count (:678-693)."""
        memo = getattr(seq, "page_hashes", None)
        tokens = seq.token_ids
        n = len(tokens)
        if memo is not None and memo[0] == n:
            return memo[1]
        ps = self.page_size
        keys = page_key_chain(tokens, ps)
        pages = [(k, tokens[ps * i: ps * (i + 1)]) for i, k in enumerate(keys)]
        if n % ps:
            pages.append((-1, tokens[ps * len(keys):]))
        seq.page_hashes = (n, pages)
        return pages

    def probe_l2_prefetch(self, seq):
        """True when L2, and only L2, can supply part of the prompt: the first
        page past the contiguous L1 match is resident in L2 (:695-722).  The
        scan resumes where the previous probe of this sequence stopped; a stale
        resume point costs a missed prefetch, never a wrong table."""
        if not self.enable_l2_cache:
            return False
        pages = self._prompt_page_hashes(seq)
        n = len(seq.token_ids)
        resume = getattr(seq, "l2_probe_resume", None)
        start = resume[1] if resume is not None and resume[0] == n else 0
        for i in range(start, len(pages) - 1):
            h, token_ids = pages[i]
            if self._find(h, token_ids) is None:
                seq.l2_probe_resume = (n, i)
                return self.l2_pool.lookup(h, token_ids) is not None
        seq.l2_probe_resume = (n, max(0, len(pages) - 1))
        return False

    @_collector_paused
    def allocate_prefill(self, seq):
        """Page table for a prompt: the contiguous L1 prefix match (never the
        last page: a sequence must run at least one token), then the L2 matches
        that follow it (staged restores), then fresh pages, keyed except the
        last (:724-782).  The L1 prefix is referenced before anything is
        allocated, so an eviction cannot hand it out again."""
        ps = self.page_size
        pages = self._prompt_page_hashes(seq)
        page_num = len(pages)

        table = array("i")
        for i in range(page_num - 1):
            p = self._find(*pages[i])
            if p is None:
                break
            self._hold(p)
            table.append(p)
        matched = len(table)
        self.hit_cnt += matched
        seq.offset += matched * ps

        if len(self.free_page_queue) + len(self.cached_pages) >= page_num - matched:
            loads = self._prefill_pages_batched(pages, matched, table)
        else:
            loads = self._prefill_pages_one_by_one(pages, matched, table)
        self.kv_page_table[seq.seq_id] = table
        if loads:
            self.l2.stage_loads(self, seq, loads)

    def _prefill_pages_batched(self, pages, matched, table):
        """Pages past the L1 match when the free and cached queues serve every
        allocation: no in-flight store is then reclaimed in between and what L2
        holds stays fixed, so taking the pages in pieces after the lookups of
        each piece gives the pages, in the order, that one lookup and one
        allocation per page give.  The restores go to the copy engine in pieces
        (L2_FIRST_PIECE pages, doubling up to L2_LOAD_CHUNK) as they are found
        (their pages pinned first), so the link starts while the rest of the
        prompt is still being walked; the flush joins them into its transfers.
        Returns the staged restores."""
        page_num = len(pages)
        loads = _StagedLoads()
        i = matched
        if self.enable_l2_cache:
            find = self.l2_pool._find
            engine = self.l2_copy_engine
            hit = True
            limit = min(L2_FIRST_PIECE, L2_LOAD_CHUNK)
            while hit and i < page_num - 1:
                srcs = []
                while i + len(srcs) < page_num - 1 and len(srcs) < limit:
                    src = find(*pages[i + len(srcs)])
                    if src is None:
                        hit = False
                        break
                    srcs.append(src)
                if not srcs:
                    break
                got = self._take_many(len(srcs))
                piece = []
                for j, src in enumerate(srcs):
                    h, token_ids = pages[i + j]
                    piece.append({"gpu_page_idx": got[j], "l2_page_idx": src, "hash": h, "token_ids": token_ids})
                self.l2.pin_loads(self, piece)
                loads.extend(piece)
                loads.handles.append(engine.load(srcs, got))
                table.extend(got)
                i += len(srcs)
                limit = min(2 * limit, L2_LOAD_CHUNK)
            loads.pinned = True
        self.l2_hit_cnt += len(loads)
        got = self._take_many(page_num - i)
        key, last = self._key_page, page_num - 1
        for j, p in enumerate(got):
            h, token_ids = pages[i + j]
            if h != -1 and i + j != last:
                key(p, h, token_ids)  # a fresh page: unkeyed, one reference
        table.extend(got)
        return loads

    def _prefill_pages_one_by_one(self, pages, matched, table):
        """Pages past the L1 match, one lookup and one allocation at a time
        (:745-782): an allocation may retire an in-flight store, which keys L2
        pages the next lookup can find."""
        page_num = len(pages)
        loads = []
        if self.enable_l2_cache:
            for i in range(matched, page_num - 1):
                h, token_ids = pages[i]
                src = self.l2_pool.lookup(h, token_ids)
                if src is None:
                    break
                loads.append(
                    {"gpu_page_idx": self.allocate_a_page(), "l2_page_idx": src, "hash": h, "token_ids": token_ids}
                )
        self.l2_hit_cnt += len(loads)
        for load in loads:
            table.append(load["gpu_page_idx"])
        for i in range(matched + len(loads), page_num):
            h, token_ids = pages[i]
            p = self.allocate_a_page()
            if h != -1 and i != page_num - 1:
                self.update_page(p, h, token_ids)
            table.append(p)
        return loads

    @_collector_paused
    def deallocate(self, seq):
        """Release every page of the sequence, suffix first, so its suffix is
        evicted before its prefix (:784-794)."""
        table = self.kv_page_table.pop(seq.seq_id, None)
        if table is None:
            return
        for p in reversed(table):
            self._drop(p)

    def may_allocate_decode(self, seq, reserve_tokens: int = 0):
        """Grow the table to cover the tokens plus ``reserve_tokens`` (:834-845)."""
        assert not seq.finished
        table = self.kv_page_table[seq.seq_id]
        while len(table) * self.page_size < len(seq.token_ids) + reserve_tokens:
            table.append(self.allocate_a_page())

    def update_page_status_and_merge_possible(self, seq):
        """When decode fills a page: key it, or, if an identical page is already
        keyed, switch the table to that page and release this one (:847-880)."""
        ps = self.page_size
        n = len(seq.token_ids)
        if n % ps:
            return
        table = self.kv_page_table[seq.seq_id]
        slot = n // ps - 1
        page = table[slot]
        token_ids = seq.token_ids[-ps:]
        prefix = self.page_idx2hash[table[slot - 1]] if slot >= 1 else -1
        h = self.compute_hash(token_ids, prefix)
        twin = -1
        for p in self.hash2page_idx_list.get(h, ()):
            if self.page_idx2token_ids[p] == token_ids:
                self.hit_cnt += 1
                twin = p
                self.ref_counts[p] += 1
                if self.ref_counts[p] == 1:
                    assert p in self.cached_pages
                    del self.cached_pages[p]
                break
        if twin != -1:
            self.ref_counts[page] -= 1
            if self.ref_counts[page] == 0:
                if self.page_idx2hash[page] != -1:
                    self.reset_page(page)
                self.free_page_queue.append(page)
            table[slot] = twin
        elif h != -1:
            self.update_page(page, h, token_ids, from_decode=True)
