"""Page ledger of the paged KV cache: which HBM pages each sequence owns, the
prefix cache over them, and the pinned-host L2 tier with its deadline-priced
transfers.

Mirrors pipeswift/engine/block_manager.py -- ``L2PagePool`` (:22-121) and
``BlockManager`` (:124-885) -- with the same public names, arguments and
behaviour.  What differs is underneath: the bytes move through the HIP
``CopyEngine`` (a blit kernel over mapped pinned memory, one launch per batch)
and the prefix-chained page keys come from one native call per prompt
(``psk_page_hash_chain``) instead of one xxhash object per page.

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
import math
import warnings
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
        self.kv_page_table: Dict[int, array] = {}
        self.kv_cache: List[torch.Tensor] = kv_cache
        self.mla_cache_tensor: torch.Tensor = mla_cache_tensor
        # The fused [L, P, 2, ps, H, D] allocation ``kv_cache`` is viewed from.
        self.kv_cache_tensor: torch.Tensor = kv_cache_tensor
        self.page_size = page_size
        self.hit_cnt = 0

        self.enable_l2_cache = l2_cache_gb > 0
        # Assumed scheduler step: converts predicted link-seconds into the
        # step count a retire deadline is expressed in.
        self.l2_step_ms = l2_step_ms
        self.l2_hit_cnt = 0
        self.l2_store_cnt = 0
        self.l2_load_cnt = 0
        self.pending_l2_stores = []
        self.pending_l2_loads = []
        self.l2_step = 0
        # Link-seconds each direction's copy stream is predicted to still owe.
        self._l2_owed_s = {"store": 0.0, "load": 0.0}
        self._l2_pending_store_requests = []
        self._l2_pending_load_requests = []
        if self.enable_l2_cache:
            # One tensor per layer stack where the layout allows it: a page of a
            # layer is then one contiguous run (:176-189).
            if self.mla_cache_tensor is not None:
                gpu_caches = [self.mla_cache_tensor]
            elif self.kv_cache_tensor is not None:
                gpu_caches = [self.kv_cache_tensor]
            else:
                gpu_caches = list(self.kv_cache)
            self.l2_num_pages = self._resolve_l2_num_pages(l2_cache_gb, gpu_caches)
            self.l2_copy_engine = copy_engine.CopyEngine(gpu_caches, self.num_pages, self.l2_num_pages)
            self.l2_pool = L2PagePool(self.l2_num_pages)
            self.l2_cost_model = self._resolve_l2_cost_model()
            self.l2_page_bytes = max(1, self._min_across_workers(copy_engine.page_bytes(gpu_caches)))
            self.l2_views = max(1, self._min_across_workers(self.l2_copy_engine.load_params.num_tensors))
        else:
            self.l2_num_pages = 0
            self.l2_page_bytes = 0
            self.l2_views = 0
            self.l2_pool = None
            self.l2_copy_engine = None
            self.l2_cost_model = None

    def __del__(self):
        engine = getattr(self, "l2_copy_engine", None)
        if engine is not None:
            engine.close()

    @classmethod
    def compute_hash(cls, token_ids, prefix: int = -1):
        return page_key(token_ids, prefix)

    # -- L2 capacity and cost model ---------------------------------------- #

    def _resolve_l2_num_pages(self, l2_cache_gb, caches):
        """Pages of the byte budget, agreed across ranks (:233-267)."""
        pb = copy_engine.page_bytes(caches)
        budget = int(l2_cache_gb * 1024**3 + 0.5)
        local = budget // pb
        if local <= 0:
            raise ValueError(
                f"L2 cache byte budget is too small: per_rank_budget={budget} bytes, page_bytes={pb}"
            )
        agreed = self._min_across_workers(local)
        if agreed < local:
            warnings.warn(
                f"L2 cache pages lowered to the minimum over ranks: local={local}, agreed={agreed}",
                RuntimeWarning,
            )
            local = agreed
        if local < self.num_pages:
            warnings.warn(
                "L2 cache holds fewer pages than the GPU pool, so only part of what L1 "
                f"evicts fits; num_pages={self.num_pages}, l2_pages={local}, "
                f"per_rank_budget={budget} bytes, page_bytes={pb}",
                RuntimeWarning,
            )
        return local

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

    def _resolve_l2_cost_model(self):
        """Per-direction integer ``{desc_rate, bw}`` from the engine's
        calibration, reduced to the minimum over ranks (:270-288)."""
        model = self.l2_copy_engine.calibrate()
        return {
            direction: {term: max(1, self._min_across_workers(int(v))) for term, v in terms.items()}
            for direction, terms in model.items()
        }

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

    def _retain_gpu_page_for_transfer(self, page_idx):
        self._hold(page_idx)

    def _release_gpu_pages_from_transfer(self, ordered_page_idxs):
        """Drop a transfer's reference on each page, in eviction order: a page
        reaching zero joins the tail of its queue (:372-387)."""
        for p in ordered_page_idxs:
            self._drop(p)

    def reset_page(self, page_idx):
        self._unkey_page(page_idx)

    def update_page(self, page_idx, h, token_ids, from_decode=False):
        """Key a page this sequence alone holds; pages completed by decode are
        also staged for L2 (:814-832)."""
        assert h != -1 and self.page_idx2hash[page_idx] == -1 and self.ref_counts[page_idx] == 1
        self._key_page(page_idx, h, token_ids)
        if from_decode and self.enable_l2_cache:
            self._stage_l2_store(page_idx, h, token_ids)

    def get_usage(self):
        return 1 - (len(self.free_page_queue) + len(self.cached_pages)) / self.num_pages

    def get_l2_usage(self):
        return self.l2_pool.get_usage() if self.enable_l2_cache else 0.0

    # -- L2 stores (GPU -> host) ------------------------------------------- #

    def _stage_l2_store(self, page_idx, h, token_ids):
        """Queue a store for the step's batched flush (:393-404)."""
        if not self.enable_l2_cache or self.l2_pool.has_page_or_pending(h, token_ids):
            return False
        key = (h, tuple(token_ids))
        self._l2_pending_store_requests.append((page_idx, h, token_ids, key))
        self.l2_pool.acquire_pending_key(key)
        return True

    def flush_l2_stores(self):
        """Send the staged stores whose page still carries the staged key (:406-418)."""
        if not self._l2_pending_store_requests:
            return 0
        staged, self._l2_pending_store_requests = self._l2_pending_store_requests, []
        live = []
        for page_idx, h, token_ids, key in staged:
            self.l2_pool.release_pending_key(key)
            if self.page_idx2hash[page_idx] == h:
                live.append((page_idx, h, token_ids))
        return self._schedule_l2_store_batch(live)

    def schedule_l2_stores_for_confirmed_seq(self, seq):
        """Store the keyed pages of the sequence's confirmed tokens (:420-431)."""
        if not self.enable_l2_cache or seq.seq_id not in self.kv_page_table:
            return
        table = self.kv_page_table[seq.seq_id]
        confirmed = min(len(seq.token_ids) // self.page_size, len(table))
        stores = []
        for p in table[:confirmed]:
            h = self.page_idx2hash[p]
            if h != -1:
                stores.append((p, h, self.page_idx2token_ids[p]))
        self._schedule_l2_store_batch(stores)

    def _schedule_l2_store_batch(self, stores):
        """One D2H transfer for every store not already resident or on its way;
        stops at the first store no L2 page can take (:433-474).

        The transfer is one logical copy, as in the reference, but it is
        submitted in pieces (L2_FIRST_PIECE pages, doubling up to
        L2_STORE_CHUNK) while this loop is still walking the batch, so the link
        starts moving the first pages instead of waiting for the host's per-page
        bookkeeping of the whole batch (about 12 ms for an 8192-page prompt).  Page ids, order and the deadline
        priced from the whole batch's runs are those of a single submission."""
        if not self.enable_l2_cache:
            return 0
        gpu, l2, keys, toks = [], [], [], []
        handles = []
        sent = 0
        pool = self.l2_pool
        engine = self.l2_copy_engine
        # pool.has_page_or_pending / acquire_pending_key and self._hold,
        # inlined with the key tuple built once: this runs once per page
        pending, find, take = pool._pending_store_keys, pool._find, pool.allocate_for_store
        rc, cached = self.ref_counts, self.cached_pages
        piece = min(L2_FIRST_PIECE, L2_STORE_CHUNK)
        for page_idx, h, token_ids in stores:
            key = (h, tuple(token_ids))
            if h != -1 and (key in pending or find(h, token_ids) is not None):
                continue
            dst = take()
            if dst is None:
                break
            # Claimed now, so a duplicate later in this batch is caught above.
            pending[key] = pending.get(key, 0) + 1
            if rc[page_idx] == 0 and page_idx in cached:
                del cached[page_idx]
            rc[page_idx] += 1
            gpu.append(page_idx)
            l2.append(dst)
            keys.append(h)
            toks.append(token_ids)
            if len(gpu) - sent >= piece:
                handles.append(engine.store(gpu[sent:], l2[sent:]))
                sent = len(gpu)
                piece = min(2 * piece, L2_STORE_CHUNK)
        if not gpu:
            return 0
        if sent < len(gpu):
            handles.append(engine.store(gpu[sent:], l2[sent:]))
        if len(handles) == 1:
            copy = handles[0]
        else:
            copy = copy_engine.JoinedCopyHandle(handles, engine.count_runs(gpu, l2), len(gpu))
        self.pending_l2_stores.append(
            {
                "copy": copy,
                "due_step": self._l2_retire_step(copy, "store"),
                "gpu_page_idxs": gpu,
                "l2_page_idxs": l2,
                "hashes": keys,
                "token_ids_list": toks,
            }
        )
        self.l2_store_cnt += len(gpu)
        return len(gpu)

    def _retire_l2_stores(self, n_ready):
        """Retire the first ``n_ready`` stores (completion is FIFO): key their L2
        pages, then drop the GPU pins suffix first (:476-491)."""
        for pending in self.pending_l2_stores[:n_ready]:
            pending["copy"].wait()
            for dst, h, token_ids in zip(pending["l2_page_idxs"], pending["hashes"], pending["token_ids_list"]):
                self.l2_pool.finish_store(dst, h, token_ids)
                self.l2_pool.release_pending_key((h, tuple(token_ids)))
            self._release_gpu_pages_from_transfer(reversed(pending["gpu_page_idxs"]))
        self.pending_l2_stores = self.pending_l2_stores[n_ready:]

    # -- L2 loads (host -> GPU) -------------------------------------------- #

    def _pin_loads(self, loads):
        """Pin both pages of each restore (_hold on both tiers, inlined: this
        runs once per restored page)."""
        rc, cached = self.ref_counts, self.cached_pages
        l2 = self.l2_pool
        rc2, cached2 = l2.ref_counts, l2.cached_pages
        for load in loads:
            g, q = load["gpu_page_idx"], load["l2_page_idx"]
            if rc[g] == 0 and g in cached:
                del cached[g]
            rc[g] += 1
            if rc2[q] == 0 and q in cached2:
                del cached2[q]
            rc2[q] += 1

    def _stage_l2_loads(self, seq, loads):
        """Queue a sequence's restore for the batched flush (:497-507).  Its
        pages are pinned here (or already, where its copies went out early), so
        nothing recycles them before the flush."""
        if not getattr(loads, "pinned", False):
            self._pin_loads(loads)
        seq.l2_load_pending = True
        self._l2_pending_load_requests.append((seq, loads))

    def flush_l2_loads(self):
        """Send the staged restores as transfers of about one scheduler step
        each, split at whole sequences (:509-548)."""
        if not self._l2_pending_load_requests:
            return 0
        staged, self._l2_pending_load_requests = self._l2_pending_load_requests, []
        total = 0
        engine = self.l2_copy_engine
        for group in self._split_l2_loads(staged):
            # pages whose copies already went out (submitted while their prompt
            # was allocated) join the transfer as they are; the rest go now
            src, dst, handles, late_src, late_dst = [], [], [], [], []
            for _, loads in group:
                early = getattr(loads, "handles", None)
                if early:
                    handles.extend(early)
                for load in loads:
                    src.append(load["l2_page_idx"])
                    dst.append(load["gpu_page_idx"])
                    if not early:
                        late_src.append(load["l2_page_idx"])
                        late_dst.append(load["gpu_page_idx"])
            if late_src:
                handles.append(engine.load(late_src, late_dst))
            # one transfer, priced from the whole group's runs as one submission
            copy = handles[0] if len(handles) == 1 else copy_engine.JoinedCopyHandle(
                handles, engine.count_runs(src, dst), len(dst))
            self.pending_l2_loads.append(
                {"copy": copy, "due_step": self._l2_retire_step(copy, "load"), "seq_loads": group}
            )
            total += len(dst)
        self.l2_load_cnt += total
        return total

    def _split_l2_loads(self, staged):
        """Greedy groups of at most one step's worth of fully scattered pages;
        a sequence larger than that goes alone (:550-567)."""
        budget = max(1, int((self.l2_step_ms / 1000) / self.l2_page_s))
        groups, cur, acc = [], [], 0
        for entry in staged:
            n = len(entry[1])
            if cur and acc + n > budget:
                groups.append(cur)
                cur, acc = [], 0
            cur.append(entry)
            acc += n
        if cur:
            groups.append(cur)
        return groups

    def _retire_l2_loads(self, n_ready):
        """Retire the first ``n_ready`` restores: key the GPU pages, unpin both
        tiers, advance each live sequence past its restored pages (:569-592)."""
        ps = self.page_size
        for pending in self.pending_l2_loads[:n_ready]:
            pending["copy"].wait()
            for seq, loads in pending["seq_loads"]:
                alive = seq.seq_id in self.kv_page_table
                for load in loads:
                    self._publish_gpu_page(load["gpu_page_idx"], load["hash"], load["token_ids"])
                    self.l2_pool.release_from_load(load["l2_page_idx"])
                # Reaches zero only for a sequence released mid-load; suffix first.
                self._release_gpu_pages_from_transfer([load["gpu_page_idx"] for load in reversed(loads)])
                if alive:
                    seq.offset += len(loads) * ps
                seq.l2_load_pending = False
        self.pending_l2_loads = self.pending_l2_loads[n_ready:]

    def reclaim_l2_store_pages(self):
        """Retire the oldest in-flight store ahead of its deadline; True if
        there was one (:594-606)."""
        if not self.pending_l2_stores:
            return False
        self._retire_l2_stores(1)
        return True

    def poll_l2_events(self, step_idx):
        """Once per scheduler step: retire every transfer whose deadline step
        has arrived (:608-615)."""
        if not self.enable_l2_cache:
            return
        self.l2_step = step_idx + 1
        if not self.pending_l2_stores and not self.pending_l2_loads:
            return
        self._retire_l2_stores(self._l2_num_due(self.pending_l2_stores))
        self._retire_l2_loads(self._l2_num_due(self.pending_l2_loads))

    def _l2_retire_step(self, copy, direction):
        """Step by which ``copy`` is due.  A direction drains serially, so the
        transfer lands after everything queued ahead of it: a water level of
        link-seconds owed, floored at the current step, plus this transfer's
        ``runs * views / desc_rate + pages * page_bytes / bw`` (:617-636)."""
        model = self.l2_cost_model[direction]
        cost_s = copy.num_runs * self.l2_views / model["desc_rate"] + copy.num_pages * self.l2_page_bytes / model["bw"]
        step_s = self.l2_step_ms / 1000
        owed_s = max(self._l2_owed_s[direction], self.l2_step * step_s) + cost_s
        self._l2_owed_s[direction] = owed_s
        return int(math.ceil(owed_s / step_s))

    def _l2_num_due(self, pendings):
        """Length of the due prefix (deadlines increase along the list)."""
        for i, pending in enumerate(pendings):
            if pending["due_step"] > self.l2_step:
                return i
        return len(pendings)

    @property
    def l2_page_s(self):
        """Link-seconds of one restored page priced fully scattered: one
        descriptor per page per view (:646-655)."""
        model = self.l2_cost_model["load"]
        return self.l2_views / model["desc_rate"] + self.l2_page_bytes / model["bw"]

    def l2_load_horizon_steps(self):
        """Steps until a restore staged now would be due: what the load water
        level still owes past the current step plus the staged, unflushed pages
        (:657-672)."""
        if not self.enable_l2_cache:
            return 0
        pages = sum(len(loads) for _, loads in self._l2_pending_load_requests)
        step_s = self.l2_step_ms / 1000
        owed_s = max(self._l2_owed_s["load"] - self.l2_step * step_s, 0.0)
        return int(math.ceil((owed_s + pages * self.l2_page_s) / step_s))

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
            self._stage_l2_loads(seq, loads)

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
                self._pin_loads(piece)
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
