"""GPU parity of ``reshape_and_cache_flash_amax`` (``psk_reshape_and_cache_amax``):
the FP8 append with per-tensor scales from the step's own K and V.  Its cache
bytes, scales and amax must equal, bit for bit, those of the two calls it
replaces -- ``cache_ops.compute_kv_scales`` then ``reshape_and_cache_flash``
with those scales -- which the append and amax tests pin to the oracle; the
config 2 case is also checked against the oracle directly.  Decode-sized
batches take the fused path (the append's waves reduce the partial maxima),
larger ones the three-launch fallback; both are covered, and so are graph
replays of the fused call."""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd import cache_ops, reshape_and_cache as rc
from tests.conftest import raw

pytestmark = pytest.mark.gpu

H, D, PS = 8, 128, 16


def _inputs(seed, n, dtype=torch.bfloat16, P=512, specials=False, zero_v=False):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(n, 6 * H * D, generator=g) * 2.0
    if specials and n > 3:
        qkv[1, H * D + 5] = float("nan")
        qkv[2, H * D + 7] = float("inf")
        qkv[3, H * D + 9] = -1e30
    if zero_v:
        qkv[:, 2 * H * D: 3 * H * D] = 0.0
    qkv = qkv.to(dtype)
    slots = torch.randperm(P * PS, generator=g)[:n].to(torch.int64)
    if n:
        slots[0] = -1  # token 0 skipped: its waves still publish the scales
        slots[5::11] = -1
    cache = torch.randint(0, 256, (P, 2, PS, H, D), generator=g, dtype=torch.uint8)  # sentinel bytes
    return qkv, slots, cache


def _run_both(dev, qkv, slots, cache):
    qd = qkv.to(dev)
    k, v = qd[:, H * D: 2 * H * D].view(-1, H, D), qd[:, 2 * H * D: 3 * H * D].view(-1, H, D)
    c1 = cache.to(dev).view(torch.float8_e4m3fn)
    c2 = cache.to(dev).view(torch.float8_e4m3fn)
    sd = slots.to(dev)
    amax1 = torch.zeros(2, dtype=torch.float32, device=dev)
    s1 = cache_ops.compute_kv_scales(k, v, amax_out=amax1)
    rc.reshape_and_cache_flash(k, v, c1[:, 0], c1[:, 1], sd, s1[0:1], s1[1:2])
    amax2 = torch.zeros(2, dtype=torch.float32, device=dev)
    s2 = rc.reshape_and_cache_flash_amax(k, v, c2[:, 0], c2[:, 1], sd, amax_out=amax2)
    torch.cuda.synchronize()
    return (c1.view(torch.uint8).cpu(), s1.cpu(), amax1.cpu()), (c2.view(torch.uint8).cpu(), s2.cpu(), amax2.cpu())


def _same(a, b):
    assert torch.equal(a[0], b[0]), "cache bytes differ"
    assert np.array_equal(a[1].numpy().view(np.uint32), b[1].numpy().view(np.uint32)), f"scales {a[1]} vs {b[1]}"
    assert np.array_equal(a[2].numpy().view(np.uint32), b[2].numpy().view(np.uint32)), f"amax {a[2]} vs {b[2]}"


def test_config2_fused_equals_two_calls_and_the_oracle(dev):
    """Config 2's decode step (128 tokens, K and V as qkv column slices): the
    fused path; also the oracle's amax scale and append."""
    qkv, slots, cache = _inputs(1201, 128)
    print("amax append: config 2 shape, fused path", flush=True)
    a, b = _run_both(dev, qkv, slots, cache)
    _same(a, b)
    key = qkv[:, H * D: 2 * H * D].contiguous().view(-1, H, D)
    val = qkv[:, 2 * H * D: 3 * H * D].contiguous().view(-1, H, D)
    ks, _ = O.amax_scale(raw(key), "bf16")
    vs, _ = O.amax_scale(raw(val), "bf16")
    assert b[1][0].item() == ks and b[1][1].item() == vs
    exp = cache.numpy().copy()
    O.reshape_and_cache(raw(key), raw(val), exp[:, 0], exp[:, 1], slots.numpy(), "bf16", "fp8", ks, vs)
    assert np.array_equal(b[0].numpy(), exp)


@pytest.mark.parametrize("n", [1, 7, 700, 1023, 1024, 3000])
def test_sizes_fused_and_fallback(dev, n):
    """Decode-sized batches (fused) up to 1023 tokens, then the fallback."""
    qkv, slots, cache = _inputs(1300 + n, n, P=max(512, n // PS + 8))
    print(f"amax append: n={n}", flush=True)
    _same(*_run_both(dev, qkv, slots, cache))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_input_dtypes(dev, dtype):
    qkv, slots, cache = _inputs(1401, 96, dtype=dtype)
    print(f"amax append: dtype={dtype}", flush=True)
    _same(*_run_both(dev, qkv, slots, cache))


def test_nan_inf_and_an_all_zero_part(dev):
    """NaN is ignored by the amax and stored by the append's NaN rule; an
    infinity makes that part's scale infinite; an all-zero V gets scale 1.0."""
    qkv, slots, cache = _inputs(1402, 64, specials=True, zero_v=True)
    print("amax append: NaN/inf K, zero V", flush=True)
    a, b = _run_both(dev, qkv, slots, cache)
    _same(a, b)
    assert b[1][0].item() == float("inf") and b[1][1].item() == 1.0 and b[2][1].item() == 0.0


def test_empty_batch_gives_unit_scales(dev):
    k = torch.empty(0, H, D, dtype=torch.bfloat16, device=dev)
    cache = torch.zeros(8, 2, PS, H, D, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    out = torch.full((2,), 7.0, device=dev)
    amax = torch.full((2,), 7.0, device=dev)
    rc.reshape_and_cache_flash_amax(k, k, cache[:, 0], cache[:, 1], torch.empty(0, dtype=torch.int64, device=dev),
                                    scales_out=out, amax_out=amax)
    torch.cuda.synchronize()
    assert out.tolist() == [1.0, 1.0] and amax.tolist() == [0.0, 0.0]
    assert int(cache.view(torch.uint8).sum()) == 0


def test_consecutive_calls_share_the_workspace(dev):
    """A large call then a small one on the same workspace: the second reads
    only its own partial maxima."""
    for seed, n in ((1501, 900), (1502, 40)):
        qkv, slots, cache = _inputs(seed, n)
        if seed == 1502:
            qkv = qkv * 0.01  # a much smaller amax than the first call's
        print(f"amax append: consecutive n={n}", flush=True)
        _same(*_run_both(dev, qkv, slots, cache))


def test_graph_replays_of_the_fused_call(dev):
    """The fused call captured once and replayed over new inputs (eager work and
    synchronizations between replays): every replay equals the two eager calls."""
    n = 128
    qkv0, slots0, cache0 = _inputs(1601, n)
    q_static = qkv0.to(dev)
    slots_static = slots0.to(dev)
    cache_static = cache0.to(dev).view(torch.float8_e4m3fn)
    scales_static = torch.zeros(2, dtype=torch.float32, device=dev)
    k = q_static[:, H * D: 2 * H * D].view(-1, H, D)
    v = q_static[:, 2 * H * D: 3 * H * D].view(-1, H, D)
    rc.reshape_and_cache_flash_amax(k, v, cache_static[:, 0], cache_static[:, 1], slots_static, scales_out=scales_static)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            rc.reshape_and_cache_flash_amax(k, v, cache_static[:, 0], cache_static[:, 1], slots_static,
                                            scales_out=scales_static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for rep, seed in enumerate((1602, 1603, 1604)):
        qkv, slots, cache = _inputs(seed, n)
        if rep == 1:
            qkv = qkv * 100.0
        print(f"amax append: graph replay {rep}", flush=True)
        q_static.copy_(qkv.to(dev))
        slots_static.copy_(slots.to(dev))
        cache_static.view(torch.uint8).copy_(cache.to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref, _ = _run_both(dev, qkv, slots, cache)
        got = (cache_static.view(torch.uint8).cpu(), scales_static.cpu(), ref[2])
        _same(ref, got)
