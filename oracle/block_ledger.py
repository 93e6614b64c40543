"""CPU oracle of the page ledger, pipeswift/engine/block_manager.py.  TEST
INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline leg, never
by the product (pipeswift_amd/block_manager.py).

A brute-force restatement of the reference's algorithm in the reference's own
order of operations, kept deliberately different in structure from the
product: flat Python lists instead of deques, ordered dicts and per-key lists,
and the ``xxhash`` package called once per page exactly as the reference calls
it (block_manager.py:220-227), instead of the product's native chain.

Where the reference's order lets one page reach two owners (a matched prefix
page recycled as a restore target, block_manager.py:741-767; a restore whose
pages are pinned only at flush, :509-548), this oracle does what the reference
does and counts the event in ``hazards`` so a test can tell those states from a
disagreement.

Pinned by: the xxhash package (the reference's own dependency) for the keys;
hand-worked scenarios in tests/test_block_ledger.py whose expected page ids,
eviction orders and deadline steps are derived on paper from the reference's
source; and ``check_invariants`` (every page in exactly one state, reference
counts equal to the holders) after every operation of the random traces.
"""

from __future__ import annotations

import math
from array import array

import numpy as np
import xxhash

DECODE_RESERVE_TOKENS = 512  # block_manager.py:19


def ref_hash(token_ids, prefix=-1):
    """block_manager.py:220-227: XXH64 (seed 0) of the little-endian 8-byte
    prefix (when not -1) then ``np.array(token_ids).tobytes()``."""
    x = xxhash.xxh64()
    if prefix != -1:
        x.update(prefix.to_bytes(8, "little"))
    x.update(np.array(token_ids).tobytes())
    return x.intdigest()


def coalesce_count(src, dst):
    """Runs after sorting by source and merging pairs that both advance by one
    (copy_engine.py:407-427)."""
    if not len(src):
        return 0
    pairs = sorted(zip(src, dst))
    runs = 1
    for (s0, d0), (s1, d1) in zip(pairs, pairs[1:]):
        if not (s1 == s0 + 1 and d1 == d0 + 1):
            runs += 1
    return runs


class Tier:
    """One page pool as flat lists.  ``free`` and ``cached`` are ordered head
    first (the head is taken or evicted first); ``index`` holds (key, page) in
    the order pages were keyed."""

    def __init__(self, num_pages, first_page=0):
        self.n = num_pages
        self.refs = [0] * num_pages
        self.free = list(range(first_page, num_pages))
        self.cached = []
        self.index = []
        self.keyof = [-1] * num_pages
        self.toks = {}

    def find(self, h, token_ids):
        if h == -1:
            return None
        for k, p in self.index:
            if k == h and self.toks[p] == token_ids:
                return p
        return None

    def key(self, p, h, token_ids):
        self.keyof[p] = h
        self.toks[p] = token_ids
        self.index.append((h, p))

    def unkey(self, p):
        assert self.refs[p] == 0
        h = self.keyof[p]
        if h != -1 and (h, p) in self.index:
            self.index.remove((h, p))
        self.keyof[p] = -1
        self.toks[p] = []

    def hold(self, p):
        if self.refs[p] == 0 and p in self.cached:
            self.cached.remove(p)
        self.refs[p] += 1

    def drop(self, p):
        self.refs[p] -= 1
        assert self.refs[p] >= 0
        if self.refs[p] == 0:
            if self.keyof[p] == -1:
                self.free.append(p)
            else:
                self.cached.append(p)

    def take(self):
        if self.free:
            p = self.free.pop(0)
        elif self.cached:
            p = self.cached.pop(0)
            self.unkey(p)
        else:
            return None
        assert self.refs[p] == 0
        self.refs[p] = 1
        return p


class RefLedger:
    """The reference BlockManager's decisions (block_manager.py:124-885) over an
    injected copy engine.  Public method names follow the reference."""

    def __init__(self, num_pages, page_size, l2_num_pages=0, engine=None, cost_model=None, page_bytes=1,
                 views=1, l2_step_ms=10.0):
        self.l1 = Tier(num_pages, first_page=1)  # :152
        self.ps = page_size
        self.tables = {}
        self.hit_cnt = 0
        self.l2 = Tier(l2_num_pages) if l2_num_pages else None
        self.pending_keys = {}
        self.engine = engine
        self.model = cost_model
        self.page_bytes = page_bytes
        self.views = views
        self.step_ms = l2_step_ms
        self.l2_step = 0
        self.owed = {"store": 0.0, "load": 0.0}
        self.staged_stores = []
        self.staged_loads = []
        self.stores = []
        self.loads = []
        self.l2_hit_cnt = self.l2_store_cnt = self.l2_load_cnt = 0
        self.hazards = 0

    @property
    def on(self):
        return self.l2 is not None

    # -- pool ---------------------------------------------------------------- #

    def free_pages(self):  # :307-309
        return len(self.l1.free) + len(self.l1.cached)

    def alloc(self):  # :327-345
        while not self.l1.free and not self.l1.cached and self.reclaim_l2_store_pages():
            pass
        p = self.l1.take()
        if p is None:
            raise RuntimeError("Out of KV Pages!")
        return p

    def release_transfer(self, pages):  # :372-387
        for p in pages:
            self.l1.drop(p)

    def update_page(self, p, h, token_ids, from_decode=False):  # :814-832
        assert h != -1 and self.l1.keyof[p] == -1 and self.l1.refs[p] == 1
        self.l1.key(p, h, token_ids)
        if from_decode and self.on:
            self.stage_store(p, h, token_ids)

    # -- L2 stores ----------------------------------------------------------- #

    def l2_known(self, h, token_ids):  # :52-58
        if h == -1:
            return False
        if (h, tuple(token_ids)) in self.pending_keys:
            return True
        return self.l2.find(h, token_ids) is not None

    def key_acquire(self, key):
        self.pending_keys[key] = self.pending_keys.get(key, 0) + 1

    def key_release(self, key):
        c = self.pending_keys.get(key, 0) - 1
        if c > 0:
            self.pending_keys[key] = c
        else:
            self.pending_keys.pop(key, None)

    def stage_store(self, p, h, token_ids):  # :393-404
        if not self.on or self.l2_known(h, token_ids):
            return False
        key = (h, tuple(token_ids))
        self.staged_stores.append((p, h, token_ids, key))
        self.key_acquire(key)
        return True

    def flush_l2_stores(self):  # :406-418
        if not self.staged_stores:
            return 0
        staged, self.staged_stores = self.staged_stores, []
        keep = []
        for p, h, t, key in staged:
            self.key_release(key)
            if self.l1.keyof[p] == h:
                keep.append((p, h, t))
        return self.store_batch(keep)

    def schedule_l2_stores_for_confirmed_seq(self, seq):  # :420-431
        if not self.on or seq.seq_id not in self.tables:
            return
        table = self.tables[seq.seq_id]
        n = min(len(seq.token_ids) // self.ps, len(table))
        self.store_batch([(p, self.l1.keyof[p], self.l1.toks[p]) for p in table[:n] if self.l1.keyof[p] != -1])

    def store_batch(self, stores):  # :433-474
        if not self.on:
            return 0
        g, l, hs, ts = [], [], [], []
        for p, h, t in stores:
            if self.l2_known(h, t):
                continue
            q = self.l2.take()
            if q is None:
                break
            if any(ld["l2_page_idx"] == q for _, lds in self.staged_loads for ld in lds):
                self.hazards += 1  # the source of a staged, unflushed restore is overwritten
            self.key_acquire((h, tuple(t)))
            self.l1.hold(p)
            g.append(p)
            l.append(q)
            hs.append(h)
            ts.append(t)
        if not g:
            return 0
        copy = self.engine.store(g, l)
        self.stores.append({"copy": copy, "due": self.due(copy, "store"), "g": g, "l": l, "h": hs, "t": ts})
        self.l2_store_cnt += len(g)
        return len(g)

    def retire_stores(self, n):  # :476-491
        for x in self.stores[:n]:
            x["copy"].wait()
            for q, h, t in zip(x["l"], x["h"], x["t"]):
                self.l2.refs[q] -= 1
                assert self.l2.refs[q] >= 0
                self.l2.key(q, h, t)
                if self.l2.refs[q] == 0:
                    self.l2.cached.append(q)
                self.key_release((h, tuple(t)))
            self.release_transfer(list(reversed(x["g"])))
        self.stores = self.stores[n:]

    # -- L2 loads ------------------------------------------------------------ #

    def flush_l2_loads(self):  # :509-548
        if not self.staged_loads:
            return 0
        staged, self.staged_loads = self.staged_loads, []
        total = 0
        for group in self.split(staged):
            src, dst = [], []
            for _, loads in group:
                for ld in loads:
                    p = ld["gpu_page_idx"]
                    if self.l1.refs[p] == 0:
                        self.hazards += 1  # target already returned to the pool
                    self.l1.hold(p)
                    self.l2.hold(ld["l2_page_idx"])
                    src.append(ld["l2_page_idx"])
                    dst.append(p)
            copy = self.engine.load(src, dst)
            self.loads.append({"copy": copy, "due": self.due(copy, "load"), "seq_loads": group})
            total += len(dst)
        self.l2_load_cnt += total
        return total

    def page_s(self):  # :646-655
        m = self.model["load"]
        return self.views / m["desc_rate"] + self.page_bytes / m["bw"]

    def split(self, staged):  # :550-567
        budget = max(1, int((self.step_ms / 1000) / self.page_s()))
        groups, cur, acc = [], [], 0
        for e in staged:
            if cur and acc + len(e[1]) > budget:
                groups.append(cur)
                cur, acc = [], 0
            cur.append(e)
            acc += len(e[1])
        if cur:
            groups.append(cur)
        return groups

    def retire_loads(self, n):  # :569-592
        for x in self.loads[:n]:
            x["copy"].wait()
            for seq, loads in x["seq_loads"]:
                alive = seq.seq_id in self.tables
                for ld in loads:
                    p = ld["gpu_page_idx"]
                    if self.l1.keyof[p] == -1:
                        self.l1.key(p, ld["hash"], ld["token_ids"])
                    self.l2.drop(ld["l2_page_idx"])
                self.release_transfer([ld["gpu_page_idx"] for ld in reversed(loads)])
                if alive:
                    seq.offset += len(loads) * self.ps
                seq.l2_load_pending = False
        self.loads = self.loads[n:]

    def reclaim_l2_store_pages(self):  # :594-606
        if not self.stores:
            return False
        self.retire_stores(1)
        return True

    def poll_l2_events(self, step_idx):  # :608-615
        if not self.on:
            return
        self.l2_step = step_idx + 1
        if not self.stores and not self.loads:
            return
        self.retire_stores(self.num_due(self.stores))
        self.retire_loads(self.num_due(self.loads))

    def due(self, copy, direction):  # :617-636
        m = self.model[direction]
        cost = copy.num_runs * self.views / m["desc_rate"] + copy.num_pages * self.page_bytes / m["bw"]
        step_s = self.step_ms / 1000
        owed = max(self.owed[direction], self.l2_step * step_s) + cost
        self.owed[direction] = owed
        return int(math.ceil(owed / step_s))

    def num_due(self, pend):  # :638-644
        for i, x in enumerate(pend):
            if x["due"] > self.l2_step:
                return i
        return len(pend)

    def l2_load_horizon_steps(self):  # :657-672
        if not self.on:
            return 0
        pages = sum(len(loads) for _, loads in self.staged_loads)
        step_s = self.step_ms / 1000
        owed = max(self.owed["load"] - self.l2_step * step_s, 0.0)
        return int(math.ceil((owed + pages * self.page_s()) / step_s))

    # -- sequences ----------------------------------------------------------- #

    def prompt_pages(self, seq):  # :678-693, recomputed every call
        ps = self.ps
        out, h = [], -1
        for i in range((len(seq.token_ids) + ps - 1) // ps):
            t = seq.token_ids[ps * i: ps * (i + 1)]
            h = ref_hash(t, h) if len(t) == ps else -1
            out.append((h, t))
        return out

    def probe_l2_prefetch(self, seq):  # :695-722, resuming where the last probe stopped
        if not self.on:
            return False
        pages = self.prompt_pages(seq)
        n = len(seq.token_ids)
        hint = getattr(seq, "l2_probe_resume", None)
        start = hint[1] if hint is not None and hint[0] == n else 0
        for i in range(start, len(pages) - 1):
            if self.l1.find(*pages[i]) is None:
                seq.l2_probe_resume = (n, i)
                return self.l2.find(*pages[i]) is not None
        seq.l2_probe_resume = (n, max(0, len(pages) - 1))
        return False

    def allocate_prefill(self, seq):  # :724-782, in the reference's order
        pages = self.prompt_pages(seq)
        n = len(pages)
        matched = []
        for i in range(n - 1):
            p = self.l1.find(*pages[i])
            if p is None:
                break
            matched.append(p)
        loads = []
        if self.on:
            for i in range(len(matched), n - 1):
                q = self.l2.find(*pages[i])
                if q is None:
                    break
                g = self.alloc()
                if g in matched:
                    self.hazards += 1  # a matched prefix page recycled as restore target
                loads.append({"gpu_page_idx": g, "l2_page_idx": q, "hash": pages[i][0], "token_ids": pages[i][1]})
        table = array("i")
        for p in matched:
            self.hit_cnt += 1
            self.l1.refs[p] += 1
            if self.l1.refs[p] == 1:
                self.l1.cached.remove(p)
            table.append(p)
        seq.offset += len(matched) * self.ps
        for ld in loads:
            self.l2_hit_cnt += 1
            table.append(ld["gpu_page_idx"])
        for i in range(len(matched) + len(loads), n):
            h, t = pages[i]
            p = self.alloc()
            if h != -1 and i != n - 1:
                self.update_page(p, h, t)
            table.append(p)
        self.tables[seq.seq_id] = table
        if loads:
            seq.l2_load_pending = True
            self.staged_loads.append((seq, loads))

    def deallocate(self, seq):  # :784-794
        table = self.tables.pop(seq.seq_id, None)
        if table is not None:
            for p in reversed(table):
                self.l1.drop(p)

    def may_allocate_decode(self, seq, reserve_tokens=0):  # :834-845
        table = self.tables[seq.seq_id]
        while len(table) * self.ps < len(seq.token_ids) + reserve_tokens:
            table.append(self.alloc())

    def update_page_status_and_merge_possible(self, seq):  # :847-880
        ps = self.ps
        n = len(seq.token_ids)
        if n % ps:
            return
        table = self.tables[seq.seq_id]
        j = n // ps - 1
        p = table[j]
        t = seq.token_ids[-ps:]
        h = ref_hash(t, self.l1.keyof[table[j - 1]] if j >= 1 else -1)
        twin = None
        for k, q in self.l1.index:
            if k == h and self.l1.toks[q] == t:
                twin = q
                break
        if twin is not None:
            self.hit_cnt += 1
            self.l1.refs[twin] += 1
            if self.l1.refs[twin] == 1:
                self.l1.cached.remove(twin)
            self.l1.refs[p] -= 1
            if self.l1.refs[p] == 0:
                if self.l1.keyof[p] != -1:
                    self.l1.unkey(p)
                self.l1.free.append(p)
            table[j] = twin
        else:
            self.update_page(p, h, t, from_decode=True)

    # -- invariants ---------------------------------------------------------- #

    def check_invariants(self):
        """Every page in exactly one state, references equal to the holders,
        keyed pages exactly the indexed ones."""
        holders = [0] * self.l1.n
        for table in self.tables.values():
            for p in table:
                holders[p] += 1
        for x in self.stores:
            for p in x["g"]:
                holders[p] += 1
        for x in self.loads:
            for _, loads in x["seq_loads"]:
                for ld in loads:
                    holders[ld["gpu_page_idx"]] += 1
        check_tier(self.l1, holders, first_page=1)
        if self.on:
            holders = [0] * self.l2.n
            for x in self.stores:
                for q in x["l"]:
                    holders[q] += 1
            for x in self.loads:
                for _, loads in x["seq_loads"]:
                    for ld in loads:
                        holders[ld["l2_page_idx"]] += 1
            check_tier(self.l2, holders, first_page=0)


def check_tier(tier, holders, first_page):
    assert tier.refs == holders, "reference counts differ from the holders"
    free, cached = set(tier.free), set(tier.cached)
    assert len(free) == len(tier.free) and len(cached) == len(tier.cached), "page queued twice"
    for p in range(first_page, tier.n):
        states = (tier.refs[p] > 0) + (p in free) + (p in cached)
        assert states == 1, f"page {p} is in {states} states"
        if p in free:
            assert tier.keyof[p] == -1, f"free page {p} is keyed"
        if p in cached:
            assert tier.keyof[p] != -1, f"cached page {p} is not keyed"
    keyed = sorted((tier.keyof[p], p) for p in range(tier.n) if tier.keyof[p] != -1)
    assert sorted(tier.index) == keyed, "index differs from the keyed pages"
