"""Graph static-metadata refresh (psk_refresh_graph_metadata, one kernel in
place of cudagraph.py:75-118's copy/fill sequence) and the next draft decode
step's metadata (psk_build_next_decode_metadata, metadata.py:351-414) on the
GPU, against the oracle restatements, with every static buffer pre-filled with
seeded sentinels so that untouched elements are checked too."""

from array import array

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd import cudagraph, metadata
from pipeswift_amd.metadata import KVCacheInfo

pytestmark = pytest.mark.gpu


def _sentinel_static(static, g):
    for name in ("page_table", "actual_lens_q", "actual_lens_kv", "cu_seqlens_q"):
        t = getattr(static, name)
        t.copy_(torch.randint(-1000, 1000, t.shape, generator=g, dtype=torch.int32))
    static.slot_mapping.copy_(torch.randint(-10**9, 10**9, static.slot_mapping.shape, generator=g,
                                            dtype=torch.int64))


def _host_static(static):
    return {"page_table": static.page_table.cpu().numpy().copy(),
            "slot_mapping": static.slot_mapping.cpu().numpy().copy(),
            "lens_q": static.actual_lens_q.cpu().numpy().copy(),
            "lens_kv": static.actual_lens_kv.cpu().numpy().copy(),
            "cu_seqlens_q": static.cu_seqlens_q.cpu().numpy().copy()}


def _step(bsz, width, pad, g, dev, strided):
    """A step's device metadata: page table [bsz, width] (optionally a column
    slice of a wider tensor), bsz * pad slots, lens_q = pad, cu_seqlens_q."""
    wide = torch.randint(0, 1 << 20, (bsz, width + (3 if strided else 0)), generator=g, dtype=torch.int32)
    pt = wide.to(dev)[:, :width]
    slots = torch.randint(-1, 1 << 30, (bsz * pad,), generator=g, dtype=torch.int64).to(dev)
    lens_q = torch.full((bsz,), pad, dtype=torch.int32, device=dev)
    lens_kv = torch.randint(1, 1 << 16, (bsz,), generator=g, dtype=torch.int32).to(dev)
    cu = torch.zeros(bsz + 1, dtype=torch.int32)
    cu[1:] = torch.arange(1, bsz + 1, dtype=torch.int32) * pad
    return KVCacheInfo(page_table=pt, slot_mapping=slots, actual_lens_q=lens_q, actual_lens_kv=lens_kv,
                       cu_seqlens_q=cu.to(dev))


def _host_step(step):
    return {"page_table": step.page_table.cpu().numpy(), "slot_mapping": step.slot_mapping.cpu().numpy(),
            "lens_q": step.actual_lens_q.cpu().numpy(), "lens_kv": step.actual_lens_kv.cpu().numpy(),
            "cu_seqlens_q": step.cu_seqlens_q.cpu().numpy()}


def _check(static, exp, what):
    got = _host_static(static)
    for k in exp:
        assert np.array_equal(got[k], exp[k]), f"{what}: {k}"


@pytest.mark.parametrize("bsz,cg_bsz,max_bsz,width,static_width,pad,strided", [
    (3, 8, 8, 4, 6, 1, False),     # padded batch, narrower step table
    (5, 5, 8, 6, 6, 1, True),      # unpadded: rows past the batch untouched
    (1, 16, 32, 1, 64, 2, False),  # two tokens per sequence (pad_q_len 2)
    (0, 4, 4, 3, 3, 1, False),     # empty batch: everything padded
    (200, 256, 512, 2048, 2048, 1, True),
])
def test_graph_refresh_matches_oracle(dev, bsz, cg_bsz, max_bsz, width, static_width, pad, strided):
    g = torch.Generator().manual_seed(bsz * 131 + cg_bsz)
    static = cudagraph.initialize_graph_kvcacheinfo(max_bsz, static_width, max_num_tokens=max_bsz * pad, device=dev)
    assert (static.slot_mapping == -1).all() and (static.cu_seqlens_q.cpu() == torch.arange(max_bsz + 1)).all()
    _sentinel_static(static, g)
    step = _step(bsz, width, pad, g, dev, strided)
    exp = O.graph_refresh(_host_static(static), _host_step(step), cg_bsz, pad)
    cudagraph.set_graph_kvcacheinfo(static, step, cg_bsz, pad_q_len=pad)
    torch.cuda.synchronize()
    _check(static, exp, f"bsz {bsz} of {cg_bsz}")


def test_graph_refresh_rejects_bad_shapes(dev):
    static = cudagraph.initialize_graph_kvcacheinfo(4, 3, device=dev)
    g = torch.Generator().manual_seed(3)
    with pytest.raises(AssertionError):
        cudagraph.set_graph_kvcacheinfo(static, _step(5, 3, 1, g, dev, False), 8)  # batch > static rows
    with pytest.raises(AssertionError):
        cudagraph.set_graph_kvcacheinfo(static, _step(2, 4, 1, g, dev, False), 4)  # wider than the static table
    with pytest.raises(AssertionError):
        cudagraph.set_graph_kvcacheinfo(static, _step(3, 3, 1, g, dev, False), 2)  # bsz > cg_bsz


def test_graph_refresh_and_append_replay_in_a_graph(dev):
    """The refresh captured together with the append that reads its static
    slot_mapping: step buffers at fixed addresses are rewritten eagerly between
    replays (with other eager work and synchronizations in between); every
    replay's static fields and cache match the oracle / the eager append."""
    from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash

    B, W, P, ps, H, D = 16, 8, 64, 16, 2, 64
    static = cudagraph.initialize_graph_kvcacheinfo(B, W, device=dev)
    g = torch.Generator().manual_seed(5)
    live = _step(B, W, 1, g, dev, False)  # fixed-address step buffers
    key = torch.zeros(B, H, D, dtype=torch.bfloat16, device=dev)
    val = torch.zeros_like(key)
    cache = torch.zeros(P, 2, ps, H, D, dtype=torch.bfloat16, device=dev)
    ref = cache.clone()
    view = KVCacheInfo(page_table=live.page_table, slot_mapping=live.slot_mapping, actual_lens_q=live.actual_lens_q,
                       actual_lens_kv=live.actual_lens_kv, cu_seqlens_q=live.cu_seqlens_q)
    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        for _ in range(2):  # warm up outside capture
            cudagraph.set_graph_kvcacheinfo(static, view, B)
            reshape_and_cache_flash(key, val, cache[:, 0], cache[:, 1], static.slot_mapping)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            cudagraph.set_graph_kvcacheinfo(static, view, B)
            reshape_and_cache_flash(key, val, cache[:, 0], cache[:, 1], static.slot_mapping)
    torch.cuda.synchronize()
    cache.zero_()
    for rep in range(4):
        fresh = _step(B, W, 1, g, dev, False)
        slots = torch.randperm(P * ps, generator=g)[:B].to(torch.int64)
        slots[rep::5] = -1
        fresh.slot_mapping.copy_(slots.to(dev))
        for name in ("page_table", "slot_mapping", "actual_lens_q", "actual_lens_kv", "cu_seqlens_q"):
            getattr(live, name).copy_(getattr(fresh, name))
        key.copy_(torch.randn(B, H, D, generator=g).to(torch.bfloat16))
        val.copy_(torch.randn(B, H, D, generator=g).to(torch.bfloat16))
        exp = O.graph_refresh(_host_static(static), _host_step(fresh), B)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check(static, exp, f"replay {rep}")
        reshape_and_cache_flash(key, val, ref[:, 0], ref[:, 1], slots.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(cache.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"


class _Seq:
    def __init__(self, seq_id, n_tokens, offset):
        self.seq_id, self.token_ids, self.offset = seq_id, list(range(n_tokens)), offset


@pytest.mark.parametrize("dcp,rank,il", [(1, 0, 1), (2, 1, 4)])
def test_next_decode_step_on_device_matches_host(dev, dcp, rank, il):
    rng = np.random.default_rng(7)
    ps, B = 16, 64
    table, rows, seqs = {}, [], []
    for b in range(B):
        n = int(rng.integers(1, 2000))
        row = rng.permutation(100000)[: (n + ps - 1) // ps].astype(np.int32)
        table[b] = array("i", row.tolist())
        rows.append(row.tolist())
        seqs.append(_Seq(b, n, n - 1))
    info = metadata.prepare_kv_info(seqs, table, ps, None, None, is_decode=True, dcp_deg=dcp, dcp_rank=rank,
                                    dcp_interleave_size=il, device=dev)
    nxt = metadata.derive_kvcache_info_next_decode_step(info, seqs, table, ps, dcp_interleave_size=il, dcp_deg=dcp,
                                                        dcp_rank=rank, device=dev)
    torch.cuda.synchronize()
    slots, lens = O.next_decode_step(rows, [s.offset for s in seqs], info.actual_lens_kv_cpu.tolist(), ps, dcp, rank,
                                     il)
    assert nxt.slot_mapping.device == dev and nxt.actual_lens_kv.device == dev
    assert nxt.slot_mapping.cpu().tolist() == slots.tolist()
    assert nxt.actual_lens_kv.cpu().tolist() == lens.tolist() == nxt.actual_lens_kv_cpu.tolist()
