"""Page ledger (pipeswift_amd.block_manager) against the reference-order oracle
(oracle/block_ledger.py), on the CPU with a copy engine that moves page tags
between two dicts instead of bytes between HBM and pinned memory.

The expected values of the hand-worked scenarios are derived on paper from
pipeswift/engine/block_manager.py (cited per step); they pin the oracle, and
the product must reproduce them too.  Random traces then compare the two
implementations state for state after every call.
"""

import math
import random
from array import array

import numpy as np
import pytest
import torch
import xxhash

from oracle import block_ledger as O
from pipeswift_amd import block_manager as BM
from pipeswift_amd import copy_engine as CE

PAGE_BYTES = 32  # kv_cache_tensor [1, P, 2, ps, 1, 16 // ps] of bytes
MODEL = {"store": {"desc_rate": 2000, "bw": 32000}, "load": {"desc_rate": 2000, "bw": 32000}}


class Seq:
    def __init__(self, seq_id, tokens):
        self.seq_id = seq_id
        self.token_ids = array("i", tokens)
        self.offset = 0
        self.finished = False
        self.l2_load_pending = False
        self.page_hashes = None
        self.l2_probe_resume = None


class Handle:
    def __init__(self, src, dst):
        self.num_pages = len(src)
        self.num_runs = O.coalesce_count(list(src), list(dst))
        self.waited = 0

    def wait(self):
        self.waited += 1


class FakeEngine:
    """Moves page tags at submit time; ``gpu[p]`` / ``host[q]`` are whatever the
    test wrote there."""

    class _Params:
        num_tensors = 1

    def __init__(self, gpu_caches=None, gpu_num_pages=0, l2_num_pages=0, **_):
        self.gpu, self.host = {}, {}
        self.load_params = self.store_params = FakeEngine._Params()
        self.calls = []
        self.closed = False

    def store(self, gpu_page_idxs, l2_page_idxs):
        for p, q in zip(gpu_page_idxs, l2_page_idxs):
            self.host[q] = self.gpu.get(p)
        self.calls.append(("store", list(gpu_page_idxs), list(l2_page_idxs)))
        return Handle(gpu_page_idxs, l2_page_idxs)

    def load(self, l2_page_idxs, gpu_page_idxs):
        for q, p in zip(l2_page_idxs, gpu_page_idxs):
            self.gpu[p] = self.host.get(q)
        self.calls.append(("load", list(l2_page_idxs), list(gpu_page_idxs)))
        return Handle(l2_page_idxs, gpu_page_idxs)

    def count_runs(self, src, dst):
        return O.coalesce_count(list(src), list(dst))

    def calibrate(self):
        return {d: dict(t) for d, t in MODEL.items()}

    def close(self):
        self.closed = True


def make_product(monkeypatch, num_pages, ps, l2_pages):
    engines = []

    def factory(*a, **k):
        engines.append(FakeEngine(*a, **k))
        return engines[-1]

    monkeypatch.setattr(CE, "CopyEngine", factory)
    cache = torch.empty(1, num_pages, 2, ps, 1, 16 // ps, dtype=torch.uint8)
    assert CE.page_bytes([cache]) == PAGE_BYTES
    gb = l2_pages * PAGE_BYTES / 1024**3
    m = BM.BlockManager(num_pages, ps, [cache[:, :, 0], cache[:, :, 1]], None, kv_cache_tensor=cache, l2_cache_gb=gb)
    assert (m.l2_num_pages if l2_pages else 0) == l2_pages
    return m, (engines[0] if engines else None)


def make_oracle(num_pages, ps, l2_pages):
    eng = FakeEngine()
    r = O.RefLedger(num_pages, ps, l2_pages, engine=eng if l2_pages else None, cost_model=MODEL,
                    page_bytes=PAGE_BYTES, views=1)
    return r, eng


# --------------------------------------------------------------------------- #
# normalized state of either implementation
# --------------------------------------------------------------------------- #


def _index(pairs):
    out = {}
    for h, p in pairs:
        out.setdefault(h, []).append(p)
    return out


def state_product(m):
    s = {
        "tables": {k: list(v) for k, v in m.kv_page_table.items()},
        "l1_free": list(m.free_page_queue),
        "l1_cached": list(m.cached_pages),
        "l1_refs": m.ref_counts.tolist(),
        "l1_keys": list(m.page_idx2hash),
        "l1_index": {h: list(v) for h, v in m.hash2page_idx_list.items()},
        "counts": (m.hit_cnt, m.l2_hit_cnt, m.l2_store_cnt, m.l2_load_cnt),
        "staged_loads": [(s.seq_id, [(ld["gpu_page_idx"], ld["l2_page_idx"]) for ld in lds])
                         for s, lds in m._l2_pending_load_requests],
    }
    if m.enable_l2_cache:
        pool = m.l2_pool
        s.update({
            "l2_free": list(pool.free_page_queue),
            "l2_cached": list(pool.cached_pages),
            "l2_refs": pool.ref_counts.tolist(),
            "l2_keys": list(pool.page_idx2hash),
            "l2_index": {h: list(v) for h, v in pool.hash2page_idx_list.items()},
            "pending_keys": dict(pool._pending_store_keys),
            "stores": [(x.gpu_page_idxs, x.l2_page_idxs, x.due_step) for x in m.pending_l2_stores],
            "loads": [(x.due_step, [(s.seq_id, [(ld["gpu_page_idx"], ld["l2_page_idx"]) for ld in lds])
                                    for s, lds in x.seq_loads]) for x in m.pending_l2_loads],
            "staged_stores": [(p, key[0]) for p, key, _ in m._l2_pending_store_requests],
            "owed": dict(m._l2_owed_s),
            "step": m.l2_step,
        })
    return s


def state_oracle(r):
    s = {
        "tables": {k: list(v) for k, v in r.tables.items()},
        "l1_free": list(r.l1.free),
        "l1_cached": list(r.l1.cached),
        "l1_refs": list(r.l1.refs),
        "l1_keys": list(r.l1.keyof),
        "l1_index": _index(r.l1.index),
        "counts": (r.hit_cnt, r.l2_hit_cnt, r.l2_store_cnt, r.l2_load_cnt),
        "staged_loads": [(s.seq_id, [(ld["gpu_page_idx"], ld["l2_page_idx"]) for ld in lds])
                         for s, lds in r.staged_loads],
    }
    if r.on:
        s.update({
            "l2_free": list(r.l2.free),
            "l2_cached": list(r.l2.cached),
            "l2_refs": list(r.l2.refs),
            "l2_keys": list(r.l2.keyof),
            "l2_index": _index(r.l2.index),
            "pending_keys": dict(r.pending_keys),
            "stores": [(x["g"], x["l"], x["due"]) for x in r.stores],
            "loads": [(x["due"], [(s.seq_id, [(ld["gpu_page_idx"], ld["l2_page_idx"]) for ld in lds])
                                  for s, lds in x["seq_loads"]]) for x in r.loads],
            "staged_stores": [(p, h) for p, h, _, _ in r.staged_stores],
            "owed": dict(r.owed),
            "step": r.l2_step,
        })
    return s


# Pages of a staged restore are pinned at staging by the product and at flush by
# the reference, so these differ until the flush.
_PIN_TIMING = ("l1_refs", "l2_refs", "l2_cached")


def assert_same(m, r):
    a, b = state_product(m), state_oracle(r)
    skip = _PIN_TIMING if b["staged_loads"] else ()
    for k in b:
        if k not in skip:
            assert a[k] == b[k], f"{k}: product {a[k]} != reference order {b[k]}"


def check_product_invariants(m):
    """The oracle's invariant check, run on the product's state."""
    tier = O.Tier(m.num_pages, first_page=1)
    tier.refs, tier.free, tier.cached = m.ref_counts.tolist(), list(m.free_page_queue), list(m.cached_pages)
    tier.keyof = list(m.page_idx2hash)
    tier.index = [(h, p) for h, ps in m.hash2page_idx_list.items() for p in ps]
    holders = [0] * m.num_pages
    for t in m.kv_page_table.values():
        for p in t:
            holders[p] += 1
    for x in m.pending_l2_stores:
        for p in x.gpu_page_idxs:
            holders[p] += 1
    staged = [lds for _, lds in m._l2_pending_load_requests] + [
        lds for x in m.pending_l2_loads for _, lds in x.seq_loads]
    for lds in staged:
        for ld in lds:
            holders[ld["gpu_page_idx"]] += 1
    O.check_tier(tier, holders, first_page=1)
    if m.enable_l2_cache:
        pool = m.l2_pool
        t2 = O.Tier(pool.num_pages)
        t2.refs, t2.free, t2.cached = pool.ref_counts.tolist(), list(pool.free_page_queue), list(pool.cached_pages)
        t2.keyof = list(pool.page_idx2hash)
        t2.index = [(h, p) for h, ps in pool.hash2page_idx_list.items() for p in ps]
        holders = [0] * pool.num_pages
        for x in m.pending_l2_stores:
            for q in x.l2_page_idxs:
                holders[q] += 1
        for lds in staged:
            for ld in lds:
                holders[ld["l2_page_idx"]] += 1
        O.check_tier(t2, holders, first_page=0)


# --------------------------------------------------------------------------- #
# page keys
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("n", [0, 1, 3, 4, 7, 8, 9, 16, 33, 64, 100, 1000])
def test_page_key_matches_xxhash(n):
    rng = np.random.default_rng(n)
    toks = array("i", rng.integers(-2**31, 2**31, n, dtype=np.int64).tolist())
    for prefix in (-1, 0, 1, 2**63 + 12345, 2**64 - 1):
        x = xxhash.xxh64()
        if prefix != -1:
            x.update(prefix.to_bytes(8, "little"))
        x.update(np.array(toks).tobytes())
        assert BM.page_key(toks, prefix) == x.intdigest() == O.ref_hash(toks, prefix)
    # a list hashes as int64, like np.array(list) in the reference
    lst = list(toks)
    assert BM.page_key(lst) == xxhash.xxh64(np.array(lst, dtype=np.int64).tobytes()).intdigest()


@pytest.mark.parametrize("n,ps", [(0, 4), (3, 4), (4, 4), (17, 4), (64, 16), (1000, 16), (4097, 256)])
def test_page_key_chain_matches_reference_loop(n, ps):
    rng = np.random.default_rng(n + ps)
    seq = Seq(0, rng.integers(0, 150000, n).tolist())
    ref = O.RefLedger(4, ps).prompt_pages(seq)
    m = BM.BlockManager(4, ps, None, None)
    got = m._prompt_page_hashes(seq)
    assert [h for h, _ in got] == [h for h, _ in ref]
    assert [list(t) for _, t in got] == [list(t) for _, t in ref]
    assert all(isinstance(t, array) for _, t in got)
    assert m._prompt_page_hashes(seq) is got  # memoized by token count
    seq.token_ids.append(5)
    assert m._prompt_page_hashes(seq) is not got


def test_page_key_chain_capacity_error():
    from pipeswift_amd._lib import lib

    toks = np.arange(16, dtype=np.int32)
    keys = np.empty(2, dtype=np.uint64)
    got = lib().psk_page_hash_chain(toks.ctypes.data, 16, 4, 4, 0, 0, keys.ctypes.data, 2)
    assert got == -4 and "do not fit" in lib().psk_last_error().decode()
    assert lib().psk_page_hash_chain(toks.ctypes.data, 16, 4, 0, 0, 0, keys.ctypes.data, 2) == -1


# --------------------------------------------------------------------------- #
# hand-worked scenarios (expected values from block_manager.py by hand)
# --------------------------------------------------------------------------- #


IMPLS = ["product", "oracle"]


def build(kind, monkeypatch, num_pages, ps, l2_pages=0):
    if kind == "product":
        m, eng = make_product(monkeypatch, num_pages, ps, l2_pages)
        return m, eng, lambda: state_product(m)
    r, eng = make_oracle(num_pages, ps, l2_pages)
    return r, eng, lambda: state_oracle(r)


@pytest.mark.parametrize("kind", IMPLS)
def test_prefix_reuse_and_suffix_first_eviction(kind, monkeypatch):
    m, _, st = build(kind, monkeypatch, 8, 2)
    a = Seq(1, [1, 2, 3, 4, 5])
    m.allocate_prefill(a)  # fresh 1, 2, 3; the last page is never keyed (:764-767)
    s = st()
    assert s["tables"][1] == [1, 2, 3] and s["l1_free"] == [4, 5, 6, 7]
    assert s["l1_keys"][1] != -1 and s["l1_keys"][2] != -1 and s["l1_keys"][3] == -1
    m.deallocate(a)  # suffix first: unkeyed 3 -> free, then 2, 1 -> cached (:784-794)
    s = st()
    assert s["l1_free"] == [4, 5, 6, 7, 3] and s["l1_cached"] == [2, 1]
    b = Seq(2, [1, 2, 3, 4, 9, 9, 7])
    m.allocate_prefill(b)  # matches pages 1, 2; fresh 4 (keyed), 5
    s = st()
    assert s["tables"][2] == [1, 2, 4, 5] and b.offset == 4 and s["counts"][0] == 2
    assert s["l1_free"] == [6, 7, 3] and s["l1_cached"] == []
    m.deallocate(b)
    assert st()["l1_cached"] == [4, 2, 1] and st()["l1_free"] == [6, 7, 3, 5]
    c = Seq(3, [6] * 9)  # 5 pages: the free queue first, then the cached head (4) is evicted
    m.allocate_prefill(c)
    s = st()
    assert s["tables"][3] == [6, 7, 3, 5, 4] and s["l1_cached"] == [2, 1] and s["l1_free"] == []
    assert s["l1_keys"][4] == -1 and all(4 not in v for v in s["l1_index"].values())
    assert m.free_pages() == 2


@pytest.mark.parametrize("kind", IMPLS)
def test_decode_page_merges_into_identical_page(kind, monkeypatch):
    m, _, st = build(kind, monkeypatch, 8, 2)
    a, b = Seq(1, [1, 2, 3]), Seq(2, [1, 2, 3])
    m.allocate_prefill(a)  # [1, 2]
    m.allocate_prefill(b)  # page 1 matched (a hit), fresh 3
    assert st()["tables"] == {1: [1, 2], 2: [1, 3]} and b.offset == 2
    for s in (a, b):
        s.token_ids.append(4)
        m.may_allocate_decode(s)
        m.update_page_status_and_merge_possible(s)  # (:847-880)
    s = st()
    # a keys page 2 with key(tokens [3, 4], prefix = key of page 1); b finds it,
    # drops its own page 3 to the free queue and switches to page 2.
    assert s["tables"] == {1: [1, 2], 2: [1, 2]}
    assert s["l1_refs"][1] == 2 and s["l1_refs"][2] == 2 and s["l1_refs"][3] == 0
    assert s["l1_free"] == [4, 5, 6, 7, 3] and s["counts"][0] == 2
    assert s["l1_keys"][2] == O.ref_hash(array("i", [3, 4]), O.ref_hash(array("i", [1, 2])))


@pytest.mark.parametrize("kind", IMPLS)
def test_l2_round_trip_deadlines(kind, monkeypatch):
    """Per page 32 B / 32000 B/s = 1 ms, per run 1 / 2000 = 0.5 ms, step 10 ms."""
    m, eng, st = build(kind, monkeypatch, 6, 2, l2_pages=4)
    a = Seq(1, [1, 2, 3, 4, 5])
    m.allocate_prefill(a)
    for i, p in enumerate(st()["tables"][1]):
        eng.gpu[p] = ("A", i)
    m.poll_l2_events(0)  # l2_step = 1
    m.schedule_l2_stores_for_confirmed_seq(a)
    s = st()
    # pages 1, 2 -> L2 0, 1 as one run: 0.5 ms + 2 ms = 2.5 ms owed past step 1's 10 ms -> due ceil(1.25) = 2
    assert s["stores"] == [([1, 2], [0, 1], 2)] and s["counts"][2] == 2
    assert s["l1_refs"][1] == 2 and s["l1_refs"][2] == 2
    assert eng.host == {0: ("A", 0), 1: ("A", 1)}
    m.deallocate(a)
    assert st()["l1_free"] == [4, 5, 3] and st()["l1_cached"] == []  # 1, 2 still pinned by the store
    m.poll_l2_events(1)  # l2_step = 2: due
    s = st()
    assert s["stores"] == [] and s["l2_cached"] == [0, 1] and s["l1_cached"] == [2, 1]
    assert s["l2_keys"][0] == s["l1_keys"][1] and s["l2_keys"][1] == s["l1_keys"][2]
    e = Seq(2, [9] * 9)  # 5 pages: 4, 5, 3, then evicts 2 and 1
    m.allocate_prefill(e)
    assert st()["tables"][2] == [4, 5, 3, 2, 1]
    m.deallocate(e)
    assert st()["l1_free"] == [1] and st()["l1_cached"] == [2, 3, 5, 4]
    b = Seq(3, [1, 2, 3, 4, 7])
    assert m.probe_l2_prefetch(b)
    m.allocate_prefill(b)  # L2 hits for pages 0, 1 -> targets 1 (free) and 2 (evicted); fresh 3
    s = st()
    assert s["tables"][3] == [1, 2, 3] and b.l2_load_pending and b.offset == 0 and s["counts"][1] == 2
    assert s["staged_loads"] == [(3, [(1, 0), (2, 1)])]
    # 2 staged pages * (0.5 + 1) ms = 3 ms -> 1 step
    assert m.l2_load_horizon_steps() == 1
    assert m.flush_l2_loads() == 2
    s = st()
    # one run: 2.5 ms owed past step 2's 20 ms -> due ceil(2.25) = 3
    assert [d for d, _ in s["loads"]] == [3] and s["counts"][3] == 2
    assert m.l2_load_horizon_steps() == 1  # 22.5 ms - 20 ms still owed
    m.poll_l2_events(1)  # step 2: not due
    assert b.l2_load_pending
    m.poll_l2_events(2)  # step 3
    s = st()
    assert not b.l2_load_pending and b.offset == 4 and s["loads"] == []
    assert eng.gpu[1] == ("A", 0) and eng.gpu[2] == ("A", 1)
    assert s["l1_keys"][1] == s["l2_keys"][0] and s["l1_refs"][1] == 1 and s["l1_refs"][2] == 1
    assert s["l2_cached"] == [0, 1] and s["l2_refs"] == [0, 0, 0, 0]


@pytest.mark.parametrize("kind", IMPLS)
def test_split_loads_into_step_sized_groups(kind, monkeypatch):
    # page_s = 1.5 ms, so one 10 ms step holds int(10 / 1.5) = 6 pages (:550-567)
    m, eng, st = build(kind, monkeypatch, 64, 2, l2_pages=40)
    seqs = []
    for i, n in enumerate([4, 3, 2, 5]):
        s = Seq(10 + i, [100 * i + k for k in range(2 * n + 1)])  # n full pages + 1
        m.allocate_prefill(s)
        m.schedule_l2_stores_for_confirmed_seq(s)
        seqs.append(s)
    m.poll_l2_events(100)
    for s in seqs:
        m.deallocate(s)
    filler = Seq(99, [7] * 2 * 63)  # evict everything from L1
    m.allocate_prefill(filler)
    m.deallocate(filler)
    twins = [Seq(20 + i, list(s.token_ids)) for i, s in enumerate(seqs)]
    for t in twins:
        m.allocate_prefill(t)
    m.flush_l2_loads()
    groups = [[sid for sid, _ in g] for _, g in st()["loads"]]
    # 4 restored pages, then 3 (4 + 3 > 6), then 2 (3 + 2 <= 6), then 5
    assert groups == [[20], [21, 22], [23]]
    assert [len(l) for _, g in st()["loads"] for _, l in g] == [4, 3, 2, 5]


def test_prefix_page_is_never_a_restore_target(monkeypatch):
    """The reference allocates restore targets before it references the matched
    L1 prefix (:741-767); with the free queue empty the LRU eviction hands the
    matched page out again.  The product references the prefix first."""
    m, meng = make_product(monkeypatch, 6, 2, 4)
    r, reng = make_oracle(6, 2, 4)
    for impl, eng in ((m, meng), (r, reng)):
        a = Seq(1, [1, 2, 3, 4, 5])
        impl.allocate_prefill(a)
        eng.gpu.update({1: "k0", 2: "k1"})
        impl.poll_l2_events(0)
        impl.schedule_l2_stores_for_confirmed_seq(a)
        impl.deallocate(a)
        impl.poll_l2_events(1)  # stores land: L1 cached [2, 1], free [4, 5, 3]
        x = Seq(2, [8] * 5)
        impl.allocate_prefill(x)  # 4, 5, 3
        impl.allocate_prefill(Seq(3, [7]))  # evicts 2 (key k1); cached [1]
        impl.deallocate(x)  # free [3], cached [1, 5, 4]
        impl.allocate_prefill(Seq(4, [6]))  # takes 3; free []
    assert_same(m, r)
    b_m, b_r = Seq(5, [1, 2, 3, 4, 6]), Seq(5, [1, 2, 3, 4, 6])
    m.allocate_prefill(b_m)
    r.allocate_prefill(b_r)
    assert r.hazards == 1 and list(r.tables[5]) == [1, 1, 5]  # page 1 is prefix and restore target
    assert list(m.kv_page_table[5]) == [1, 5, 4]
    check_product_invariants(m)
    m.flush_l2_loads()
    m.poll_l2_events(10)
    assert meng.gpu[1] == "k0" and meng.gpu[5] == "k1" and b_m.offset == 4
    r.flush_l2_loads()
    r.poll_l2_events(10)
    assert reng.gpu[1] == "k1"  # the reference's prefix page now holds the restored page


def test_staged_restore_source_survives_a_store_batch(monkeypatch):
    """Between staging (allocate_prefill) and flush, the reference leaves the L2
    source unpinned (:509-548); a store batch in between can evict it and
    overwrite its bytes.  The product pins it at staging."""
    m, meng = make_product(monkeypatch, 12, 2, 2)
    r, reng = make_oracle(12, 2, 2)
    out = {}
    for name, impl, eng in (("product", m, meng), ("oracle", r, reng)):
        a = Seq(1, [1, 2, 3])
        impl.allocate_prefill(a)  # page 1 (keyed), page 2
        eng.gpu[1] = "a0"
        impl.poll_l2_events(0)
        impl.schedule_l2_stores_for_confirmed_seq(a)  # page 1 -> L2 0
        impl.deallocate(a)
        impl.poll_l2_events(5)  # L2 cached [0]
        filler = Seq(2, [9] * 21)  # 11 pages: evicts page 1 from L1
        impl.allocate_prefill(filler)
        impl.deallocate(filler)
        c = Seq(3, [5, 6, 7, 8, 1])
        impl.allocate_prefill(c)
        for i, p in enumerate((impl.kv_page_table if name == "product" else impl.tables)[3][:2]):
            eng.gpu[p] = f"c{i}"
        b = Seq(4, [1, 2, 3])
        impl.allocate_prefill(b)  # restore of L2 0 staged, not yet flushed
        impl.schedule_l2_stores_for_confirmed_seq(c)  # wants 2 L2 pages; L2 holds 2
        impl.flush_l2_loads()
        impl.poll_l2_events(50)
        tb = (impl.kv_page_table if name == "product" else impl.tables)[4]
        out[name] = eng.gpu[tb[0]]
    assert out["product"] == "a0"
    assert out["oracle"] == "c1"  # the reference restored the page that evicted its source
    check_product_invariants(m)


def test_public_helpers(monkeypatch):
    m, _ = make_product(monkeypatch, 100, 16, 8)
    s = Seq(1, list(range(40)))
    assert m.decode_reserve_pages(3) == 3 * 32
    assert m.can_allocate(s) and m.can_allocate(s, reserve_tokens=16 * 96)
    assert not m.can_allocate(s, reserve_tokens=16 * 97)
    m.allocate_prefill(s)
    assert m.get_usage() == pytest.approx(1 - 96 / 100) and m.get_l2_usage() == 0.0
    assert m.can_allocate_overlap_schedule([s])  # (40 + 16) // 16 = 3 pages held already
    assert m.l2_page_s == pytest.approx(1 / 2000 + 32 / 32000)
    with pytest.raises(ValueError):
        BM.BlockManager(4, 16, None, None, l2_step_ms=0)
    off = BM.BlockManager(4, 16, None, None)
    assert not off.enable_l2_cache and off.l2_load_horizon_steps() == 0 and not off.probe_l2_prefetch(s)
    off.poll_l2_events(3)
    assert off.flush_l2_stores() == 0 and off.flush_l2_loads() == 0
    with pytest.raises(RuntimeError, match="Out of KV Pages"):
        for _ in range(4):
            off.allocate_a_page()


def test_allocate_drains_in_flight_stores_before_failing(monkeypatch):
    """A store pins the GPU pages it reads; a full pool retires the oldest store
    early rather than failing (:327-345, :594-606)."""
    m, eng = make_product(monkeypatch, 4, 2, 4)
    a = Seq(1, [1, 2, 3, 4, 5])  # pages 1, 2 (keyed), 3
    m.allocate_prefill(a)
    m.schedule_l2_stores_for_confirmed_seq(a)
    m.deallocate(a)  # 1, 2 pinned by the store; 3 free
    m.allocate_prefill(Seq(2, [9]))  # takes 3
    assert m.free_pages() == 0 and len(m.pending_l2_stores) == 1
    p = m.allocate_a_page()  # retires the store: cached [2, 1], evicts 2
    assert not m.pending_l2_stores and p == 2 and list(m.cached_pages) == [1]


@pytest.mark.parametrize("kind", IMPLS)
def test_restore_lookup_after_an_allocation_that_retires_a_store(kind, monkeypatch):
    """With both queues empty the prompt's first restore target comes from
    retiring the in-flight store, and that store keys the L2 page the next
    lookup then finds: lookups and allocations must interleave page by page
    (:741-767, :327-345).  Looking every page up before allocating would stage
    one restore instead of two."""
    m, _, st = build(kind, monkeypatch, 8, 2, l2_pages=8)
    a = Seq(1, [1, 2, 3])  # page 1 = [1, 2] keyed, page 2 partial
    m.allocate_prefill(a)
    m.poll_l2_events(0)
    m.schedule_l2_stores_for_confirmed_seq(a)  # page 1 -> L2 0
    m.poll_l2_events(5)  # retired: L2 0 resident
    m.deallocate(a)
    assert st()["l1_free"] == [3, 4, 5, 6, 7, 2] and st()["l1_cached"] == [1]
    b = Seq(2, [1, 2, 3, 4, 5, 6, 7, 8, 9])  # L1 hit on page 1, then 3, 4, 5 keyed, 6 partial
    m.allocate_prefill(b)
    assert st()["tables"][2] == [1, 3, 4, 5, 6]
    m.schedule_l2_stores_for_confirmed_seq(b)  # [1, 2] already in L2; 3, 4, 5 -> L2 1, 2, 3 in flight
    assert [(g, l) for g, l, _ in st()["stores"]] == [([3, 4, 5], [1, 2, 3])]
    m.deallocate(b)  # 3, 4, 5 stay pinned by the store
    assert st()["l1_free"] == [7, 2, 6] and st()["l1_cached"] == [1]
    d = Seq(3, [50] * 7)  # 4 pages: the 3 free ones, then evicts 1
    m.allocate_prefill(d)
    s = st()
    assert s["tables"][3] == [7, 2, 6, 1] and s["l1_free"] == [] and s["l1_cached"] == []
    c = Seq(4, [1, 2, 3, 4, 0])
    m.allocate_prefill(c)
    # page 0: L2 hit on L2 0; its target retires the store (L1 cached [5, 4, 3])
    # and takes 5; page 1: now an L2 hit on L2 1, target 4; partial page: 3
    s = st()
    assert s["stores"] == [] and s["tables"][4] == [5, 4, 3]
    assert s["staged_loads"] == [(4, [(5, 0), (4, 1)])] and s["counts"][1] == 2
    assert m.flush_l2_loads() == 2


# --------------------------------------------------------------------------- #
# random traces: product and reference-order oracle, call for call
# --------------------------------------------------------------------------- #


def run_trace(monkeypatch, seed, steps=600, num_pages=32, ps=4, l2_pages=64, admit_past_free=0.0):
    """Random calls on the product and the reference-order oracle, comparing
    every state.  A fraction ``admit_past_free`` of the prompts is admitted
    whatever the free count, so allocation may have to retire in-flight stores
    part-way through a prompt; the trace ends at the first out-of-pages error,
    which both must raise."""
    rng = random.Random(seed)
    m, _ = make_product(monkeypatch, num_pages, ps, l2_pages)
    r, _ = make_oracle(num_pages, ps, l2_pages)
    docs = [[rng.randrange(40) for _ in range(80)] for _ in range(3)]
    live = {}
    step, next_id, compared = 0, 0, 0
    for _ in range(steps):
        op = rng.random()
        if op < 0.22:
            d = rng.choice(docs)
            n = rng.randrange(1, 48)
            cut = rng.randrange(0, n + 1)
            toks = d[:cut] + [rng.randrange(40) for _ in range(n - cut)]
            need = (n + ps - 1) // ps
            # past the free count only as far as in-flight stores pin pages
            pinned = sum(len(x.gpu_page_idxs) for x in m.pending_l2_stores)
            past_free = rng.random() < admit_past_free and m.free_pages() + pinned >= need
            if not past_free and m.free_pages() < need:
                continue
            pa, ra = Seq(next_id, toks), Seq(next_id, toks)
            next_id += 1
            assert m.probe_l2_prefetch(pa) == r.probe_l2_prefetch(ra)
            try:
                m.allocate_prefill(pa)
            except RuntimeError as e:
                assert past_free and "Out of KV Pages" in str(e)
                with pytest.raises(RuntimeError, match="Out of KV Pages"):
                    r.allocate_prefill(ra)
                break
            r.allocate_prefill(ra)
            live[pa.seq_id] = (pa, ra)
            if rng.random() < 0.7:  # the scheduler flushes restores right after admitting them
                assert m.flush_l2_loads() == r.flush_l2_loads()
        elif op < 0.50 and live:
            pa, ra = live[rng.choice(sorted(live))]
            if pa.l2_load_pending:
                continue
            need = len(m.kv_page_table[pa.seq_id]) * ps <= len(pa.token_ids)
            if need and m.free_pages() == 0:
                continue
            t = rng.randrange(40)
            for s in (pa, ra):
                s.token_ids.append(t)
            m.may_allocate_decode(pa)
            r.may_allocate_decode(ra)
            m.update_page_status_and_merge_possible(pa)
            r.update_page_status_and_merge_possible(ra)
        elif op < 0.60 and live:
            pa, ra = live[rng.choice(sorted(live))]
            m.schedule_l2_stores_for_confirmed_seq(pa)
            r.schedule_l2_stores_for_confirmed_seq(ra)
        elif op < 0.68:
            assert m.flush_l2_stores() == r.flush_l2_stores()
        elif op < 0.76:
            assert m.l2_load_horizon_steps() == r.l2_load_horizon_steps()
            assert m.flush_l2_loads() == r.flush_l2_loads()
        elif op < 0.88:
            step += rng.randrange(1, 3)
            m.poll_l2_events(step)
            r.poll_l2_events(step)
        elif op < 0.97 and live:
            sid = rng.choice(sorted(live))
            pa, ra = live[sid]
            if any(s is pa for s, _ in m._l2_pending_load_requests):
                continue
            m.deallocate(pa)
            r.deallocate(ra)
            del live[sid]
        else:
            assert m.reclaim_l2_store_pages() == r.reclaim_l2_store_pages()
        if r.hazards:
            break  # the reference order has handed a page to two owners
        assert_same(m, r)
        for pa, ra in live.values():
            assert (pa.offset, pa.l2_load_pending) == (ra.offset, ra.l2_load_pending)
        r.check_invariants()
        check_product_invariants(m)
        compared += 1
    return compared, m


@pytest.mark.parametrize("seed", range(16))
def test_random_trace_matches_reference_order(seed, monkeypatch):
    # A trace stops comparing at the reference's first double-owner state.
    compared, m = run_trace(monkeypatch, seed)
    assert compared >= 60
    assert m.l2_store_cnt > 0 and m.hit_cnt > 0


def test_random_traces_exercise_restores(monkeypatch):
    runs = [run_trace(monkeypatch, seed) for seed in range(16)]
    assert sum(c for c, _ in runs) > 6000
    assert sum(m.l2_load_cnt for _, m in runs) > 200 and sum(m.l2_hit_cnt for _, m in runs) > 200


@pytest.mark.parametrize("seed", range(6))
def test_random_trace_with_store_batches_submitted_in_pieces(seed, monkeypatch):
    """A store batch goes to the copy engine in pieces of L2_STORE_CHUNK pages
    while the ledger walks it; with pieces of 2 pages every ledger state,
    deadline and page id still equals the reference order's (one submission)."""
    monkeypatch.setattr(BM, "L2_STORE_CHUNK", 2)
    compared, m = run_trace(monkeypatch, seed)
    assert compared >= 60 and m.l2_store_cnt > 0


def test_random_trace_admitting_past_the_free_pages(monkeypatch):
    """Prompts admitted past the free count take the page-by-page path of
    allocate_prefill, where an allocation retires an in-flight store; the
    short prompts of the other traces take the batched path.  Both match the
    reference order state for state."""
    paths = {"batched": 0, "one_by_one": 0, "one_by_one_reclaimed": 0}
    for name in ("batched", "one_by_one"):
        orig = getattr(BM.BlockManager, "_prefill_pages_" + name)

        def counted(self, *a, _orig=orig, _name=name):
            before = len(self.pending_l2_stores)
            out = _orig(self, *a)  # counts only calls that returned
            paths[_name] += 1
            if _name == "one_by_one" and len(self.pending_l2_stores) < before:
                paths["one_by_one_reclaimed"] += 1
            return out

        monkeypatch.setattr(BM.BlockManager, "_prefill_pages_" + name, counted)
    compared = [run_trace(monkeypatch, seed, num_pages=24, admit_past_free=0.6)[0] for seed in range(24)]
    assert sum(compared) > 2000
    assert paths["one_by_one_reclaimed"] >= 5 and paths["batched"] >= 200, paths


def test_random_traces_with_restores_submitted_while_allocating(monkeypatch):
    """Restores go to the copy engine in pieces of L2_LOAD_CHUNK pages while
    allocate_prefill walks the prompt, and the flush joins them into its
    transfers; with pieces of 2 pages every ledger state, deadline and page id
    still equals the reference order's (one submission per transfer, at the
    flush), and the restored tags land where the reference's do."""
    monkeypatch.setattr(BM, "L2_LOAD_CHUNK", 2)
    runs = [run_trace(monkeypatch, seed) for seed in range(12)]
    assert sum(c for c, _ in runs) > 4000
    assert sum(m.l2_load_cnt for _, m in runs) > 150
    loads = [c for _, m in runs for c in m.l2_copy_engine.calls if c[0] == "load"]
    # every restored page went out exactly once, in pieces of at most 2 pages
    assert loads and all(len(c[1]) <= 2 for c in loads)
    staged = sum(len(lds) for _, m in runs for _, lds in m._l2_pending_load_requests)
    assert sum(len(c[1]) for c in loads) == sum(m.l2_load_cnt for _, m in runs) + staged


def test_ledger_walks_pause_the_collector_and_restore_its_state():
    """The bulk walks (prefill allocation, store scheduling, restore flush,
    release) run with Python's cyclic collector held off and leave it as they
    found it: enabled after a walk, enabled after a walk that raised, and
    still disabled when it was disabled before."""
    import gc

    from pipeswift_amd import block_manager as bm

    for name in ("allocate_prefill", "schedule_l2_stores_for_confirmed_seq", "flush_l2_loads", "deallocate"):
        assert getattr(getattr(bm.BlockManager, name), "__wrapped__", None) is not None, name
    seen = []

    @bm._collector_paused
    def walk(fail=False):
        seen.append(gc.isenabled())
        if fail:
            raise RuntimeError("walk failed")
        return 5

    was = gc.isenabled()
    try:
        gc.enable()
        assert walk() == 5 and seen[-1] is False and gc.isenabled()
        with pytest.raises(RuntimeError):
            walk(fail=True)
        assert seen[-1] is False and gc.isenabled()
        gc.disable()
        assert walk() == 5 and seen[-1] is False and not gc.isenabled()
    finally:
        (gc.enable if was else gc.disable)()
