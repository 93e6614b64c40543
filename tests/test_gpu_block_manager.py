"""The page ledger on the GPU: a prefix stored to L2 through the HIP CopyEngine,
evicted from HBM, and restored by a later prompt with the same tokens must come
back byte for byte, for each cache layout BlockManager hands the engine
(block_manager.py:176-189)."""

from array import array

import numpy as np
import pytest
import torch

from pipeswift_amd.block_manager import BlockManager
from tests.conftest import raw

pytestmark = pytest.mark.gpu


class Seq:
    def __init__(self, seq_id, tokens):
        self.seq_id = seq_id
        self.token_ids = array("i", tokens)
        self.offset = 0
        self.finished = False
        self.l2_load_pending = False
        self.page_hashes = None
        self.l2_probe_resume = None


def _layout(kind, L, P, ps, dev):
    """(kv_cache, mla_cache_tensor, kv_cache_tensor, the tensors holding page data)"""
    if kind == "fused":
        t = torch.zeros(L, P, 2, ps, 8, 128, dtype=torch.bfloat16, device=dev)
        return [t[:, :, 0], t[:, :, 1]], None, t, [t]
    if kind == "split":
        k = torch.zeros(L, P, ps, 8, 128, dtype=torch.bfloat16, device=dev)
        v = torch.zeros(L, P, ps, 8, 128, dtype=torch.bfloat16, device=dev)
        return [k, v], None, None, [k, v]
    t = torch.zeros(L, P, ps, 576, dtype=torch.bfloat16, device=dev)
    return None, t, None, [t]


def _fill(tensors, pages, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.tensor(pages, dtype=torch.int64, device=tensors[0].device)
    for t in tensors:
        shape = list(t.shape)
        shape[1] = len(pages)
        t.index_copy_(1, idx, torch.randn(shape, generator=g).to(t.dtype).to(t.device))


def _pages(tensors, pages):
    idx = torch.tensor(pages, dtype=torch.int64, device=tensors[0].device)
    return [raw(t.index_select(1, idx)) for t in tensors]


def _run_until(m, done, step, limit=10000):
    """Advance the scheduler clock until ``done()``; every transfer retires by
    its deadline step, which is finite."""
    while not done():
        step += 1
        assert step < limit, "transfer never came due"
        m.poll_l2_events(step)
    return step


@pytest.mark.parametrize("kind", ["fused", "split", "mla"])
def test_l2_store_evict_restore_round_trip(kind, dev):
    L, P, ps, l2_pages = 3, 80, 16, 48
    kv, mla, fused, data = _layout(kind, L, P, ps, dev)
    page_bytes = sum(t[:, 0].numel() * t.element_size() for t in data)
    m = BlockManager(P, ps, kv, mla, kv_cache_tensor=fused, l2_cache_gb=l2_pages * page_bytes / 1024**3)
    assert m.l2_num_pages == l2_pages and m.l2_page_bytes == page_bytes
    assert m.l2_views == L * len(data)  # one view per (tensor, layer)
    for d in ("store", "load"):
        assert 1e9 <= m.l2_cost_model[d]["bw"] <= 2e11, m.l2_cost_model
        assert m.l2_cost_model[d]["desc_rate"] >= 1

    rng = np.random.default_rng(5)
    prompt = rng.integers(0, 150000, 20 * ps + 7).tolist()  # 20 full pages + 7 tokens
    a = Seq(1, prompt)
    m.allocate_prefill(a)
    table_a = list(m.kv_page_table[1])
    _fill(data, table_a, seed=11)
    torch.cuda.synchronize()
    want = _pages(data, table_a[:20])

    m.poll_l2_events(0)
    m.schedule_l2_stores_for_confirmed_seq(a)
    assert m.l2_store_cnt == 20 and m.pending_l2_stores[0].due_step >= 1
    step = _run_until(m, lambda: not m.pending_l2_stores, 0)
    m.deallocate(a)

    filler = Seq(2, [7] * (ps * (P - 1)))  # every page of the pool: A's pages are evicted
    m.allocate_prefill(filler)
    _fill(data, list(m.kv_page_table[2]), seed=12)
    m.deallocate(filler)
    assert all(m._lookup_cached_page(h, t) is None for h, t in m._prompt_page_hashes(Seq(9, prompt)))

    b = Seq(3, prompt)
    assert m.probe_l2_prefetch(b)
    m.allocate_prefill(b)
    table_b = list(m.kv_page_table[3])
    assert m.l2_hit_cnt == 20 and b.l2_load_pending and b.offset == 0
    assert m.flush_l2_loads() == 20
    _run_until(m, lambda: not b.l2_load_pending, step)
    assert b.offset == 20 * ps
    got = _pages(data, table_b[:20])
    for w, g in zip(want, got):
        assert np.array_equal(w, g)
    # restored pages are keyed again, so a third copy of the prompt hits in HBM
    c = Seq(4, prompt)
    m.allocate_prefill(c)
    assert list(m.kv_page_table[4])[:20] == table_b[:20] and c.offset == 20 * ps
    m.deallocate(b)
    m.deallocate(c)
    m.l2_copy_engine.close()


def test_decode_pages_are_staged_and_flushed_once_per_step(dev):
    """Pages completed by decode are staged (update_page from_decode) and sent as
    one transfer per flush; a duplicate key is never stored twice."""
    L, P, ps = 2, 64, 16
    t = torch.zeros(L, P, 2, ps, 8, 128, dtype=torch.bfloat16, device=dev)
    page_bytes = t[:, 0].numel() * 2
    m = BlockManager(P, ps, [t[:, :, 0], t[:, :, 1]], None, kv_cache_tensor=t, l2_cache_gb=32 * page_bytes / 1024**3)
    seqs = [Seq(i, [1000 * i + k for k in range(ps - 1)]) for i in range(4)]
    for s in seqs:
        m.allocate_prefill(s)
    m.poll_l2_events(0)
    for s in seqs:  # each decode token completes the sequence's first page
        s.token_ids.append(5)
        m.may_allocate_decode(s)
        m.update_page_status_and_merge_possible(s)
    assert len(m._l2_pending_store_requests) == 4 and not m.pending_l2_stores
    assert m.flush_l2_stores() == 4 and len(m.pending_l2_stores) == 1
    _run_until(m, lambda: not m.pending_l2_stores, 0)
    assert m.l2_store_cnt == 4 and m.get_l2_usage() == pytest.approx(4 / 32)
    m.schedule_l2_stores_for_confirmed_seq(seqs[0])  # already resident: nothing sent
    assert m.l2_store_cnt == 4 and not m.pending_l2_stores
    m.l2_copy_engine.close()
