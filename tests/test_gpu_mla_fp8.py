"""GPU parity of the tile-scaled FP8 MLA entry (append and gather) with the CPU
oracle: bit-exact bytes for the append, bit-exact bf16 (and f32 up to NaN
payloads) for the gather, through the C ABI."""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
import workloads
from pipeswift_amd import impl_utils, metadata, mla_fp8
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def _f32_equal(a_bits, b_bits):
    a = a_bits.view(np.float32)
    b = b_bits.view(np.float32)
    return np.array_equal(a, b, equal_nan=True) and np.array_equal(np.isnan(a), np.isnan(b))


@pytest.mark.parametrize("decode", [False, True])
def test_config4_append_whole_cache(dev, decode):
    case = workloads.config4_mla_fp8_tiles(decode=decode)
    n = case.slot_mapping.shape[0]
    print(f"mla fp8 tiles: N={n} cache={tuple(case.cache.shape)}", flush=True)
    latent_d = case.latent.to(dev)
    k_pe_d = case.k_pe(latent_d)
    assert k_pe_d.stride(0) == 2112
    cache_d = case.cache.to(dev)
    mla_fp8.concat_and_cache_mla_fp8_tiles(case.kv_c.to(dev), k_pe_d, cache_d, case.slot_mapping.to(dev))
    exp = case.cache.numpy().copy()
    O.concat_and_cache_mla_tiles(raw(case.kv_c), raw(case.k_pe()), exp, case.slot_mapping.numpy())
    got = raw(cache_d)
    assert np.array_equal(got, exp)
    # the scales really differ from tile to tile
    s = got.reshape(-1, 656)[:, 512:528].copy().view(np.float32)
    assert len(np.unique(s)) > 100


@pytest.mark.parametrize("n,P", [(300, 40), (1500, 120)])
def test_slots_and_special_values(dev, n, P):
    """Zero, NaN, infinite, tiny and overflowing tiles, skipped and
    out-of-range slots; 1500 tokens take the prefill launch, which writes
    each entry with one store."""
    g = torch.Generator().manual_seed(41)
    ps = 16
    x = torch.randn(n, 512, generator=g) * torch.exp2(torch.randint(-20, 20, (n, 1), generator=g).float())
    x[0, :128] = 0.0                      # zero tile
    x[1, 200] = float("nan")
    x[2, 300] = float("inf")
    x[2, 301] = float("-inf")
    x[3, 400:512] = 1e-38                 # below the scale floor
    x[4, 5] = -float("nan")
    x[5] = 3.4e38                         # bf16 rounds this to +inf
    kv_c = x.to(torch.bfloat16)
    k_pe = torch.randn(n, 64, generator=g).to(torch.bfloat16)
    slots = torch.randperm(P * ps, generator=g)[:n].to(torch.int64)
    slots[6::11] = -1
    slots[7::29] = P * ps + 3             # out of range: skipped
    cache = workloads.sentinel((P, ps, 656), torch.uint8, 42)
    cd = cache.to(dev)
    mla_fp8.concat_and_cache_mla_fp8_tiles(kv_c.to(dev), k_pe.to(dev), cd, slots.to(dev))
    exp = cache.numpy().copy()
    O.concat_and_cache_mla_tiles(raw(kv_c), raw(k_pe), exp, slots.numpy())
    assert np.array_equal(raw(cd), exp)


@pytest.mark.parametrize("nope,rope,pe_off,ps,layered", [
    (128, 0, 0, 16, False),
    (256, 2, 0, 5, False),       # 268-byte entries, 4-byte aligned; block size not a power of two
    (384, 6, 1, 16, False),      # k_pe rows on 2-byte boundaries: 2-byte rope vectors
    (640, 64, 0, 64, True),      # 5 tiles (two passes), 788-byte entries; a layer of a 4-D cache
    (512, 64, 3, 64, True),
    (8192, 512, 0, 2, False),    # the largest nope (16 passes) and rope
])
def test_sizes_alignments_layouts(dev, nope, rope, pe_off, ps, layered):
    g = torch.Generator().manual_seed(43 + nope + rope)
    n, P = 97, 30
    E = mla_fp8.entry_bytes(nope, rope)
    assert E == O.mla_tile_entry_bytes(nope, rope)
    kv_c = (torch.randn(n, nope, generator=g) * 7).to(torch.bfloat16)
    proj = torch.randn(n, rope + pe_off + 5, generator=g).to(torch.bfloat16)
    k_pe = proj[:, pe_off: pe_off + rope]
    slots = torch.randperm(P * ps, generator=g)[:n].to(torch.int64)
    slots[::9] = -1
    if layered:
        full = workloads.sentinel((3, P, ps, 1, E), torch.uint8, 44)
        fd = full.to(dev)
        target = fd[1]
    else:
        full = workloads.sentinel((P, ps, E), torch.uint8, 44)
        fd = full.to(dev)
        target = fd
    print(f"sizes: nope={nope} rope={rope} pe_off={pe_off} ps={ps} layered={layered}", flush=True)
    kd = proj.to(dev)
    mla_fp8.concat_and_cache_mla_fp8_tiles(kv_c.to(dev), kd[:, pe_off: pe_off + rope], target, slots.to(dev))
    exp = full.numpy().copy()
    view = exp[1, :, :, 0] if layered else exp
    O.concat_and_cache_mla_tiles(raw(kv_c), raw(k_pe), view, slots.numpy())
    assert np.array_equal(raw(fd), exp)


def _filled_cache(dev, P, ps, seed):
    g = torch.Generator().manual_seed(seed)
    n = P * ps
    kv_c = (torch.randn(n, 512, generator=g) * torch.exp2(torch.randint(-6, 6, (n, 1), generator=g).float()))
    kv_c = kv_c.to(torch.bfloat16)
    kv_c[5, 3] = float("nan")
    k_pe = torch.randn(n, 64, generator=g).to(torch.bfloat16)
    slots = torch.randperm(n, generator=g).to(torch.int64)
    cd = torch.zeros(P, ps, 656, dtype=torch.uint8, device=dev)
    mla_fp8.concat_and_cache_mla_fp8_tiles(kv_c.to(dev), k_pe.to(dev), cd, slots.to(dev))
    return cd, kv_c, k_pe, slots


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gather_matches_oracle(dev, out_dtype):
    P, ps = 64, 64
    cd, *_ = _filled_cache(dev, P, ps, 45)
    g = torch.Generator().manual_seed(46)
    lens = [1, 64, 200, 0, 1000, 77]
    starts = [0, 64, 5, 0, 128, 0]
    W = 20
    bt = torch.randint(0, P, (len(lens), W), generator=g, dtype=torch.int32)
    bt[2, 1] = P + 5          # out of range: zero rows
    bt[4, 3] = -2
    cu = torch.tensor(np.r_[0, np.cumsum(lens)], dtype=torch.int32)
    T = int(cu[-1]) + 9       # rows past the last sequence stay untouched
    od = torch.full((T, 576), 7.0, dtype=out_dtype, device=dev)
    st = torch.tensor(starts, dtype=torch.int32)
    mla_fp8.gather_mla_fp8_tiles(cd, od, bt.to(dev), cu.to(dev), seq_starts=st.to(dev))
    exp = raw(torch.full((T, 576), 7.0, dtype=out_dtype)).copy()
    code = "bf16" if out_dtype == torch.bfloat16 else "f32"
    O.gather_mla_tiles(raw(cd), bt.numpy(), cu.numpy(), 512, seq_starts=st.numpy(), out=exp, out_dtype=code)
    got = raw(od)
    if out_dtype == torch.bfloat16:
        assert np.array_equal(got, exp)
    else:
        assert _f32_equal(got, exp)


def test_config4_round_trip_within_quantization_error(dev):
    """append then gather of the whole prefill batch: every element within half
    an E4M3 step of its tile scale, the rope part exact."""
    case = workloads.config4_mla_fp8_tiles(decode=False)
    n = case.slot_mapping.shape[0]
    P, ps = case.cache.shape[0], case.cache.shape[1]
    cd = case.cache.to(dev)
    latent_d = case.latent.to(dev)
    mla_fp8.concat_and_cache_mla_fp8_tiles(case.kv_c.to(dev), case.k_pe(latent_d), cd, case.slot_mapping.to(dev))
    # the prefill slots fill whole pages in order, so one sequence's table is the block list
    blocks = (case.slot_mapping[::ps] // ps).to(torch.int32)
    assert torch.equal(case.slot_mapping, (blocks.repeat_interleave(ps).long() * ps + torch.arange(n) % ps))
    od = torch.empty(n, 576, dtype=torch.float32, device=dev)
    mla_fp8.gather_mla_fp8_tiles(cd, od, blocks[None].to(dev), torch.tensor([0, n], dtype=torch.int32, device=dev))
    back = od.cpu().double().numpy()
    x = case.kv_c.double().numpy()
    s = np.repeat(raw(cd).reshape(P * ps, 656)[case.slot_mapping.numpy(), 512:528].copy().view(np.float32), 128,
                  axis=1).astype(np.float64)
    bound = s * np.maximum(2.0 ** -4 * np.abs(x) / s, 2.0 ** -10) * (1 + 2.0 ** -16)
    assert np.all(np.abs(back[:, :512] - x) <= bound)
    assert np.array_equal(back[:, 512:], case.k_pe().double().numpy())


def test_append_replays_in_a_hip_graph(dev):
    P, ps, n = 50, 64, 128
    g = torch.Generator().manual_seed(47)
    kv_static = torch.zeros(n, 512, dtype=torch.bfloat16, device=dev)
    pe_static = torch.zeros(n, 64, dtype=torch.bfloat16, device=dev)
    slot_static = torch.full((n,), -1, dtype=torch.int64, device=dev)
    cd = torch.zeros(P, ps, 656, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream(dev)
    with torch.cuda.stream(s):
        mla_fp8.concat_and_cache_mla_fp8_tiles(kv_static, pe_static, cd, slot_static)
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            mla_fp8.concat_and_cache_mla_fp8_tiles(kv_static, pe_static, cd, slot_static)
    exp = np.zeros((P, ps, 656), np.uint8)
    for rep in range(3):
        kv = (torch.randn(n, 512, generator=g) * (rep + 1)).to(torch.bfloat16)
        pe = torch.randn(n, 64, generator=g).to(torch.bfloat16)
        sl = torch.randperm(P * ps, generator=g)[:n].to(torch.int64)
        kv_static.copy_(kv)
        pe_static.copy_(pe)
        slot_static.copy_(sl)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        O.concat_and_cache_mla_tiles(raw(kv), raw(pe), exp, sl.numpy())
        assert np.array_equal(raw(cd), exp), rep


def test_append_mla_kv_cache_routes_a_uint8_cache(dev):
    L, P, ps, n = 2, 100, 64, 150
    cache = workloads.sentinel((L, P, ps, 656), torch.uint8, 48)
    cd = cache.to(dev)
    g = torch.Generator().manual_seed(49)
    latent = torch.randn(n, 1536 + 576, generator=g).to(torch.bfloat16)
    ckv = torch.randn(n, 512, generator=g).to(torch.bfloat16)
    slots = torch.randperm(P * ps, generator=g)[:n].to(torch.int64)
    slots[::7] = -1
    info = metadata.KVCacheInfo(mla_cache_tensor=cd, slot_mapping=slots.to(dev))
    ld = latent.to(dev)
    impl_utils.append_mla_kv_cache(ckv.to(dev), ld[:, 2048:], info, layer_idx=1)
    exp = cache.numpy().copy()
    O.concat_and_cache_mla_tiles(raw(ckv), raw(latent[:, 2048:]), exp[1], slots.numpy())
    assert np.array_equal(raw(cd), exp)


def test_argument_errors(dev):
    kv = torch.zeros(4, 512, dtype=torch.bfloat16, device=dev)
    pe = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev)
    sl = torch.zeros(4, dtype=torch.int64, device=dev)
    with pytest.raises(AssertionError, match="entry of 576 bytes"):
        mla_fp8.concat_and_cache_mla_fp8_tiles(kv, pe, torch.zeros(2, 4, 576, dtype=torch.uint8, device=dev), sl)
    with pytest.raises(AssertionError, match="bf16"):
        mla_fp8.concat_and_cache_mla_fp8_tiles(kv.half(), pe.half(), torch.zeros(2, 4, 656, dtype=torch.uint8,
                                                                                  device=dev), sl)
    base = torch.zeros(4 * 513 + 8, dtype=torch.bfloat16, device=dev)
    odd = base[1: 1 + 4 * 513].view(4, 513)[:, :512]  # rows on 2-byte boundaries
    with pytest.raises(AssertionError, match="16-byte"):
        mla_fp8.concat_and_cache_mla_fp8_tiles(odd, pe, torch.zeros(2, 4, 656, dtype=torch.uint8, device=dev), sl)
