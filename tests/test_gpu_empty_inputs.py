"""Zero-size inputs through every device entry point: the reference's callers
return early on an empty batch (impl_utils.py:304-305, 318-319), so each op must
be a no-op that leaves its outputs untouched (and, for the scales, report the
all-zero tensor's scale 1.0) without launching work on empty buffers."""

import numpy as np
import pytest
import torch

import workloads
from pipeswift_amd import attention, cache_ops
from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash_diffkv
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def test_empty_mla_append_leaves_cache_untouched(dev):
    cache = workloads.sentinel((8, 64, 1, 576), torch.bfloat16, 51).to(dev)
    before = raw(cache).copy()
    kv_c = torch.empty(0, 1, 512, dtype=torch.bfloat16, device=dev)
    k_pe = torch.empty(0, 1, 64, dtype=torch.bfloat16, device=dev)
    reshape_and_cache_flash_diffkv(kv_c, k_pe, cache, torch.empty(0, dtype=torch.int64, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(raw(cache), before)


def test_empty_gather_batches(dev):
    cache = workloads.sentinel((16, 16, 4, 128), torch.bfloat16, 52).to(dev)
    out = torch.full((5, 4, 128), 7, dtype=torch.bfloat16, device=dev)
    before = raw(out).copy()
    bt = torch.zeros(3, 4, dtype=torch.int32, device=dev)
    # no sequences, then sequences that are all empty
    cache_ops.gather_cache(cache, out, bt[:0], torch.zeros(1, dtype=torch.int32, device=dev))
    cache_ops.gather_cache(cache, out, bt, torch.zeros(4, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(raw(out), before)


def test_empty_copy_blocks_mapping(dev):
    stack = workloads.sentinel((2, 8, 2, 16, 2, 64), torch.bfloat16, 53).to(dev)
    before = raw(stack).copy()
    cache_ops.copy_blocks(stack, torch.empty(0, 2, dtype=torch.int64, device=dev))
    cache_ops.copy_blocks(stack, torch.empty(0, 2, dtype=torch.int64))
    torch.cuda.synchronize()
    assert np.array_equal(raw(stack), before)


def test_kv_scales_of_zero_tokens_is_one(dev):
    k = torch.empty(0, 8, 128, dtype=torch.bfloat16, device=dev)
    sc = cache_ops.compute_kv_scales(k, k.clone())
    assert sc.cpu().tolist() == [1.0, 1.0]


def test_decode_attention_with_no_sequences(dev):
    cache = torch.zeros(4, 16, 2, 128, dtype=torch.float8_e4m3fn, device=dev)
    q = torch.empty(0, 4, 128, dtype=torch.bfloat16, device=dev)
    out = torch.empty(0, 4, 128, dtype=torch.bfloat16, device=dev)
    bt = torch.zeros(0, 2, dtype=torch.int32, device=dev)
    lens = torch.zeros(0, dtype=torch.int32, device=dev)
    got = attention.paged_decode_attention(q, cache, cache, bt, lens, 128 ** -0.5, out=out)
    torch.cuda.synchronize()
    assert got.shape == (0, 4, 128)
