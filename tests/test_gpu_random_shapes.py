"""Seeded random-shape parity sweeps of the append, MLA concat, gather,
copy_blocks and L2 page transport entry points against the CPU oracle.

Each case draws its geometry (heads, head size, block size, pool size, token
count across the decode-sized and prefill-sized launches), dtypes, strides and
slot or block-table patterns from its seed, fills every destination with
seeded sentinel bytes, and compares the whole destination buffer byte for
byte, so a write outside the rows the oracle writes fails as surely as a wrong
row.  Slots are unique (the reference leaves duplicate slots to the order of
its program instances), and each sweep mixes -1 padding and out-of-range
entries into the slots or block tables.
"""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
import workloads
from pipeswift_amd import cache_ops
from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash, reshape_and_cache_flash_diffkv
from tests.conftest import raw

pytestmark = pytest.mark.gpu

TORCH = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "fp8": torch.float8_e4m3fn}


def _values(shape, dtype, gen, std=2.0):
    return (torch.randn(shape, generator=gen) * std).to(TORCH[dtype])


def _slots(rng, n, capacity):
    """n unique slots of [0, capacity), about 5 % -1 and 2 % past the pool."""
    n_real = min(n, capacity)
    s = np.full(n, -1, np.int64)
    s[:n_real] = rng.permutation(capacity)[:n_real]
    rng.shuffle(s)
    s[rng.random(n) < 0.05] = -1
    s[rng.random(n) < 0.02] = capacity + int(rng.integers(0, 100))
    return torch.from_numpy(s)


@pytest.mark.parametrize("seed", range(24))
def test_random_appends(dev, seed):
    rng = np.random.default_rng(1000 + seed)
    g = torch.Generator().manual_seed(1000 + seed)
    in_dt = ["bf16", "f16", "f32"][seed % 3]
    fp8 = seed % 2 == 1
    H = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 96, 128, 256]))
    ps = int(rng.choice([1, 5, 16, 32, 64]))
    N = int(rng.choice([1, 7, 128, 600, 1100, 3000]))
    P = max(2, int(np.ceil(N / ps * rng.uniform(1.1, 2.0))))
    extra = int(rng.choice([0, H * D, 8]))  # qkv row padding: key/value are strided views
    cache_dt = "fp8" if fp8 else in_dt
    print(f"append seed={seed}: {in_dt}->{cache_dt} N={N} H={H} D={D} ps={ps} P={P} extra={extra}", flush=True)
    row = 2 * H * D + extra
    qkv = _values((N, row), in_dt, g)
    key = qkv[:, :H * D].view(N, H, D)
    value = qkv[:, H * D: 2 * H * D].view(N, H, D)
    fused = workloads.sentinel((P, 2, ps, H, D), TORCH[cache_dt], 2000 + seed)
    slots = _slots(rng, N, P * ps)
    qkv_d, fused_d = qkv.to(dev), fused.to(dev)
    kd, vd = qkv_d[:, :H * D].view(N, H, D), qkv_d[:, H * D: 2 * H * D].view(N, H, D)
    ks = vs = None
    k_scale = v_scale = None
    if fp8:
        ks, vs = float(np.float32(rng.uniform(0.05, 3.0))), float(np.float32(rng.uniform(0.05, 3.0)))
        k_scale = torch.tensor([ks], dtype=torch.float32, device=dev)
        v_scale = torch.tensor([vs], dtype=torch.float32, device=dev)
    reshape_and_cache_flash(kd, vd, fused_d[:, 0], fused_d[:, 1], slots.to(dev), k_scale, v_scale)
    exp = raw(fused).copy()
    O.reshape_and_cache(raw(key.contiguous()), raw(value.contiguous()), exp[:, 0], exp[:, 1], slots.numpy(), in_dt,
                        cache_dt, ks, vs)
    assert np.array_equal(raw(fused_d), exp)


@pytest.mark.parametrize("seed", range(10))
def test_random_mla_appends(dev, seed):
    rng = np.random.default_rng(3000 + seed)
    g = torch.Generator().manual_seed(3000 + seed)
    fp8 = seed % 2 == 1
    Lk = int(rng.choice([128, 256, 512]))
    Lv = int(rng.choice([32, 64]))
    ps = int(rng.choice([1, 16, 64, 100]))
    N = int(rng.choice([1, 128, 1500, 4096]))
    P = max(2, int(np.ceil(N / ps * rng.uniform(1.1, 1.6))))
    stride = Lk + Lv + int(rng.choice([0, 64, 1536]))  # k_pe is a strided view, as transformer.py slices it
    print(f"mla seed={seed}: fp8={fp8} N={N} Lk={Lk} Lv={Lv} ps={ps} P={P} stride={stride}", flush=True)
    latent = _values((N, stride), "bf16", g)
    kv_c = latent[:, :Lk].contiguous()
    cache = workloads.sentinel((P, ps, Lk + Lv), torch.float8_e4m3fn if fp8 else torch.bfloat16, 4000 + seed)
    slots = _slots(rng, N, P * ps)
    lat_d, cache_d = latent.to(dev), cache.to(dev)
    k_pe_d = lat_d[:, Lk: Lk + Lv]
    sc = float(np.float32(rng.uniform(0.02, 2.0))) if fp8 else None
    reshape_and_cache_flash_diffkv(kv_c.to(dev).unsqueeze(1), k_pe_d.unsqueeze(1), cache_d.unsqueeze(2), slots.to(dev),
                                   None if sc is None else torch.tensor([sc], dtype=torch.float32, device=dev))
    exp = raw(cache).copy()
    O.concat_and_cache_mla(raw(kv_c), raw(latent[:, Lk: Lk + Lv].contiguous()), exp, slots.numpy(), "bf16",
                           "fp8" if fp8 else "bf16", sc)
    assert np.array_equal(raw(cache_d), exp)


@pytest.mark.parametrize("seed", range(16))
def test_random_gathers(dev, seed):
    rng = np.random.default_rng(5000 + seed)
    g = torch.Generator().manual_seed(5000 + seed)
    dequant = seed % 4 == 3
    H = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 128]))
    ps = int(rng.choice([1, 7, 16, 64]))
    B = int(rng.choice([1, 3, 40, 90]))
    lens = rng.integers(0, int(rng.choice([20, 400, 3000])), B)
    lens[rng.random(B) < 0.1] = 0
    starts = rng.integers(0, 3 * ps, B).astype(np.int32) if seed % 2 else None
    maxpos = int((lens + (0 if starts is None else starts)).max()) if B else 1
    W = maxpos // ps + 2
    P = max(W + 1, int(rng.integers(W + 1, 4 * W + 8)))
    bt = rng.integers(0, P, (B, W)).astype(np.int32)
    bad = rng.random((B, W)) < 0.02
    bt[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -1, P + 5)
    cu = np.zeros(B + 1, np.int32)
    cu[1:] = np.cumsum(lens)
    T = int(cu[-1]) + int(rng.integers(0, 20))
    pad = int(rng.choice([0, 0, 64]))
    row = H * D
    out_dt = ["bf16", "f16", "f32"][seed % 3] if dequant else "bf16"
    print(f"gather seed={seed}: B={B} T={T} H={H} D={D} ps={ps} P={P} W={W} starts={starts is not None} "
          f"dequant={dequant}->{out_dt} pad={pad}", flush=True)
    if dequant:
        caches = [torch.randint(0, 256, (P, ps, H, D), generator=g, dtype=torch.uint8) for _ in range(2)]
        for c in caches:
            c[(c & 0x7F) == 0x7F] = 0x33  # no NaN codes: NaN payloads are not pinned
        src = [c.to(dev).view(torch.float8_e4m3fn) for c in caches]
        scale = float(np.float32(rng.uniform(0.1, 4.0)))
    else:
        caches = [workloads.sentinel((P, ps, H, D), torch.bfloat16, 6000 + seed + i) for i in range(2)]
        src = [c.to(dev) for c in caches]
        scale = None
    fill = torch.full((T, row + pad), 3, dtype=TORCH[out_dt])
    full = [fill.to(dev) for _ in range(2)]
    outs = [f[:, :row].view(T, H, D) for f in full]
    cache_ops.gather_cache(src[0], outs[0], torch.from_numpy(bt).to(dev), torch.from_numpy(cu).to(dev),
                           seq_starts=None if starts is None else torch.from_numpy(starts).to(dev),
                           scale=None if scale is None else torch.tensor([scale], dtype=torch.float32, device=dev),
                           src_cache_v=src[1], dst_v=outs[1])
    for cache, f in zip(caches, full):
        exp = raw(fill).copy()
        body = exp[:, :row].reshape(T, H, D).copy()
        if dequant:
            body = O.gather_cache(cache.numpy(), bt, cu, seq_starts=starts, out=body, cache_dtype="fp8",
                                  out_dtype=out_dt, scale=scale)
        else:
            body = O.gather_cache(raw(cache), bt, cu, seq_starts=starts, out=body)
        exp[:, :row] = body.reshape(T, row)
        assert np.array_equal(raw(f), exp)


@pytest.mark.parametrize("seed", range(8))
def test_random_copy_blocks(dev, seed):
    rng = np.random.default_rng(7000 + seed)
    L = int(rng.choice([1, 3, 8]))
    P = int(rng.choice([16, 200, 1024]))
    shape = [(2, 16, 8, 128), (2, 16, 4, 64), (16, 576), (2, 5, 3, 40)][seed % 4]
    dt = [torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.float8_e4m3fn][seed % 4]
    n = int(rng.integers(1, P // 2 + 1))
    perm = rng.permutation(P)
    pairs = torch.from_numpy(np.stack([perm[:n], perm[n: 2 * n]], 1).astype(np.int64))
    print(f"copy_blocks seed={seed}: L={L} P={P} slab={shape} {dt} pairs={n}", flush=True)
    stack = workloads.sentinel((L, P) + shape, dt, 8000 + seed)
    sd = stack.to(dev)
    cache_ops.copy_blocks(sd, pairs.to(dev) if seed % 2 else pairs)
    exp = raw(stack).copy()
    O.copy_blocks(exp, pairs.numpy())
    assert np.array_equal(raw(sd), exp)


def _page_ids(rng, n, limit):
    """n unique page ids of [0, limit): runs of consecutive ids mixed with
    scattered ones, so the transfer coalesces some pages and not others."""
    out, used = [], set()
    while len(out) < n:
        start = int(rng.integers(0, limit))
        run = int(rng.choice([1, 1, 2, 5, 17]))
        for p in range(start, min(limit, start + run)):
            if p not in used and len(out) < n:
                used.add(p)
                out.append(p)
    return np.array(out, np.int64)


@pytest.mark.parametrize("seed", range(8))
def test_random_swaps(dev, seed):
    """CopyEngine store (device -> pinned host) then load (host -> other device
    pages) over one or two layered caches of different page sizes."""
    from pipeswift_amd import copy_engine

    rng = np.random.default_rng(9000 + seed)
    L = int(rng.choice([1, 2, 5]))
    P, P2 = int(rng.integers(20, 300)), int(rng.integers(20, 300))
    shapes = [[(2, 16, 2, 64), (16, 576), (2, 5, 3, 40)][seed % 3]]
    if seed % 2:
        shapes.append((8, 72))
    transport = "blit" if seed % 4 < 3 else "memcpy"
    n = int(rng.integers(1, min(P, P2) + 1))
    print(f"swap seed={seed}: L={L} P={P} P2={P2} shapes={shapes} n={n} {transport}", flush=True)
    caches = [workloads.sentinel((L, P) + sh, torch.bfloat16, 9100 + seed + i) for i, sh in enumerate(shapes)]
    cds = [c.to(dev) for c in caches]
    eng = copy_engine.CopyEngine(cds, P, P2, transport=transport)
    try:
        gpu_ids, l2_ids = _page_ids(rng, n, P), _page_ids(rng, n, P2)
        eng.store(gpu_ids.tolist(), l2_ids.tolist()).wait()
        for c, hc in zip(caches, eng.host_caches):
            assert np.array_equal(raw(hc)[:, l2_ids], raw(c)[:, gpu_ids])
        back = _page_ids(rng, n, P)
        for cd in cds:
            cd.zero_()
        eng.load(l2_ids.tolist(), back.tolist()).wait()
        untouched = np.setdiff1d(np.arange(P), back)
        for c, cd in zip(caches, cds):
            got = raw(cd)
            assert np.array_equal(got[:, back], raw(c)[:, gpu_ids])
            assert not got[:, untouched].any()
    finally:
        eng.close()
