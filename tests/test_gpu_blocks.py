"""GPU parity of copy_blocks and of the L2 page transport (swap_blocks)."""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
import workloads
from pipeswift_amd import cache_ops, copy_engine
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def test_copy_blocks_whole_stack_bit_exact(dev):
    L, P = 4, 1024
    stack = workloads.sentinel((L, P, 2, 16, 8, 128), torch.bfloat16, 41)
    pairs = workloads.config5a_pairs(num_pairs=300, num_blocks=P)
    sd = stack.to(dev)
    cache_ops.copy_blocks(sd, pairs)
    exp = raw(stack).copy()
    O.copy_blocks(exp, pairs.numpy())
    assert np.array_equal(raw(sd), exp)


def test_copy_blocks_list_of_caches_device_mapping_and_odd_slab(dev):
    """Two caches (MLA-like 576-wide rows of 9 slots: a slab that is not a
    multiple of 16 bytes) with a device-resident mapping."""
    a = workloads.sentinel((3, 50, 9, 577), torch.bfloat16, 42)
    b = workloads.sentinel((3, 50, 2, 4, 8), torch.float8_e4m3fn, 43)
    pairs = torch.tensor([[0, 49], [7, 8], [20, 1]], dtype=torch.int64)
    ad, bd = a.to(dev), b.to(dev)
    cache_ops.copy_blocks([ad, bd], pairs.to(dev))
    ea, eb = raw(a).copy(), raw(b).copy()
    O.copy_blocks(ea, pairs.numpy())
    O.copy_blocks(eb, pairs.numpy())
    assert np.array_equal(raw(ad), ea) and np.array_equal(raw(bd), eb)


def test_copy_blocks_rejects_overlap_and_range(dev):
    stack = torch.zeros(2, 10, 4, dtype=torch.bfloat16, device=dev)
    with pytest.raises(AssertionError):
        cache_ops.copy_blocks(stack, torch.tensor([[1, 2], [2, 3]]))
    with pytest.raises(AssertionError):
        cache_ops.copy_blocks(stack, torch.tensor([[1, 10]]))


def test_copy_blocks_config5a_full_size_pattern(dev):
    """61 layers x 8192 blocks (31 GiB): each (layer, block) slab holds a value
    derived from its own coordinates, so after the copy every slab must hold
    the value of (layer, expected source).  Checked on the device."""
    L, P = 61, 8192
    pairs = workloads.config5a_pairs()
    stack = torch.empty((L, P, 2, 16, 8, 128), dtype=torch.bfloat16, device=dev)
    flat = stack.view(L, P, -1).view(torch.int16)
    tag = (torch.arange(L, device=dev, dtype=torch.int32).view(L, 1) * P
           + torch.arange(P, device=dev, dtype=torch.int32).view(1, P))
    flat.copy_((tag % 32749).to(torch.int16).view(L, P, 1).expand(L, P, flat.shape[2]))
    flat[:, :, -1] = (tag // 32749).to(torch.int16)
    cache_ops.copy_blocks(stack, pairs)
    src_of = torch.arange(P, device=dev)
    src_of[pairs[:, 1].to(dev)] = pairs[:, 0].to(dev)
    exp_tag = (torch.arange(L, device=dev, dtype=torch.int32).view(L, 1) * P + src_of.view(1, P).int())
    assert torch.equal(flat[:, :, 0], (exp_tag % 32749).to(torch.int16))
    assert torch.equal(flat[:, :, 8191], (exp_tag % 32749).to(torch.int16))
    assert torch.equal(flat[:, :, -1], (exp_tag // 32749).to(torch.int16))
    assert bool((flat[:, :, :-1] == flat[:, :, :1]).all())
    del stack, flat


# --------------------------------------------------------------------------- #
# CopyEngine
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("transport", ["blit", "memcpy"])
def test_copy_engine_round_trip(dev, transport):
    L, P, P2 = 3, 96, 64
    cache = workloads.sentinel((L, P, 2, 16, 2, 64), torch.bfloat16, 44)
    cd = cache.to(dev)
    eng = copy_engine.CopyEngine([cd], P, P2, transport=transport)
    try:
        rng = np.random.default_rng(45)
        gpu_ids = rng.permutation(P)[:40]
        l2_ids = np.concatenate([np.arange(10, 30), rng.permutation(np.arange(30, 64))[:20]])
        h = eng.store(gpu_ids.tolist(), l2_ids.tolist())
        h.wait()
        host = raw(eng.host_caches[0])
        src = raw(cache)
        assert np.array_equal(host[:, l2_ids], src[:, gpu_ids])
        assert h.num_pages == 40 and h.num_runs < 40
        # load them back somewhere else on the GPU
        back = rng.permutation(P)[:40]
        cd.zero_()
        h2 = eng.load(l2_ids.tolist(), back.tolist())
        h2.wait()
        got = raw(cd)
        assert np.array_equal(got[:, back], src[:, gpu_ids])
        untouched = np.setdiff1d(np.arange(P), back)
        assert not got[:, untouched].any()
        with pytest.raises(AssertionError, match="not pages of the gpu tier"):
            eng.store([P], [0])
        with pytest.raises(AssertionError, match="not pages of the l2 tier"):
            eng.load([-1], [0])
        assert eng.load([], []).pending is False
    finally:
        eng.close()


def test_copy_engine_calibrate_and_page_bytes(dev):
    cache = torch.zeros(2, 600, 2, 16, 2, 64, dtype=torch.bfloat16, device=dev)
    assert copy_engine.page_bytes([cache]) == 2 * 2 * 16 * 2 * 64 * 2
    eng = copy_engine.CopyEngine([cache], 600, 600)
    try:
        model = eng.calibrate(num_pages=512)
        assert set(model) == {"store", "load"}
        for d in model.values():
            assert d["bw"] > 1e8 and d["desc_rate"] >= 1
        assert eng.load_params.num_tensors == 2
    finally:
        eng.close()


def test_config5b_swap_round_trip_checksum(dev):
    """8192 scattered blocks of an 8-layer [P, 2, 16, 8, 128] stack (4 GiB)
    device -> pinned host -> device, compared by per-page checksum."""
    L, Pg, P2 = 8, 16384, 8192
    gpu_ids, l2_ids = workloads.config5b_pages(gpu_pages=Pg, l2_pages=P2)
    cache = torch.empty((L, Pg, 2, 16, 8, 128), dtype=torch.bfloat16, device=dev)
    g = torch.Generator(device=dev).manual_seed(46)
    cache.view(torch.int16).random_(-32768, 32767, generator=g)
    eng = copy_engine.CopyEngine([cache], Pg, P2)
    try:
        words = cache.view(L, Pg, -1).view(torch.int32)
        def page_sums(ids):
            idx = torch.as_tensor(ids, device=dev)
            w = words[:, idx].to(torch.int64)
            return (w * torch.arange(1, w.shape[2] + 1, device=dev)).sum(dim=2)
        before = page_sums(gpu_ids)
        eng.store(gpu_ids.tolist(), l2_ids.tolist()).wait()
        cache.zero_()
        back = np.sort(gpu_ids)[::-1].copy()
        eng.load(l2_ids.tolist(), back.tolist()).wait()
        after = page_sums(back)
        assert torch.equal(before, after)
    finally:
        eng.close()
