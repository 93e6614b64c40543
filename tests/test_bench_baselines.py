"""The bench's torch CPU baselines (the reference's host path: index_put_ and
index_select) must compute what the oracle computes, or their GB/s would time
different work.  CPU only."""

import numpy as np
import torch

import bench
from oracle import kv_oracle as O
import workloads


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_torch_append_baseline_matches_oracle_bf16():
    case = workloads.config1_append(seed=5, num_tokens=200, num_blocks=64)
    step, cache = bench.torch_cpu_append_step(case, fp8=False)
    step()
    exp = np.zeros(tuple(case.cache.shape), np.uint16)
    O.reshape_and_cache(_u16(case.key()), _u16(case.value()), exp[:, 0], exp[:, 1], case.slot_mapping.numpy())
    assert np.array_equal(_u16(cache), exp)


def test_torch_append_baseline_matches_oracle_fp8():
    case = workloads.config2_fp8_decode(batch=32, num_blocks=4096, ctx_hi=2048)
    step, cache = bench.torch_cpu_append_step(case, fp8=True)
    step()
    key, value = _u16(case.key()), _u16(case.value())
    ks, _ = O.amax_scale(key, "bf16")
    vs, _ = O.amax_scale(value, "bf16")
    exp = np.zeros(tuple(case.cache.shape), np.uint8)
    O.reshape_and_cache(key, value, exp[:, 0], exp[:, 1], case.slot_mapping.numpy(), "bf16", "fp8", ks, vs)
    assert np.array_equal(cache.view(torch.uint8).numpy(), exp)


def test_torch_gather_baseline_matches_oracle():
    cc = workloads.config3_chunked(max_prefix=2000, num_blocks=2048)
    step, out = bench.torch_cpu_gather_step(cc)
    step()
    bt, cu = cc.block_table.numpy(), cc.cu_seq_lens.numpy()
    assert np.array_equal(_u16(out[0]), O.gather_cache(_u16(cc.append.cache[:, 0]), bt, cu))
    assert np.array_equal(_u16(out[1]), O.gather_cache(_u16(cc.append.cache[:, 1]), bt, cu))


def test_timed_launch_count_is_exactly_the_requested_steps():
    """The bench captures exactly --steps launches (the driver runs --steps 20;
    an earlier version replayed only whole 64-launch graphs and timed none)."""
    for rotate in (1, 4, 8, 512):
        for steps in (1, 5, 20, 63, 64, 65, 127, 2048):
            sets = bench.launch_sets(steps, rotate)
            assert len(sets) == steps
            assert sets == [i % rotate for i in range(steps)]
    assert bench.launch_sets(0, 8) == []


def test_torch_mla_baseline_matches_oracle():
    case = workloads.config4_mla(num_tokens=64, num_blocks=100, decode=True)
    step, cache = bench.torch_cpu_mla_step(case, None)
    step()
    exp = np.zeros(tuple(case.cache.shape), np.uint16)
    O.concat_and_cache_mla(_u16(case.kv_c), _u16(case.k_pe()), exp, case.slot_mapping.numpy())
    assert np.array_equal(_u16(cache), exp)
