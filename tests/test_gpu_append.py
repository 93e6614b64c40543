"""GPU parity of the paged append (MHA/GQA), bf16 and fused FP8, vs the CPU oracle.

Every comparison covers the whole cache: it is pre-filled with seeded
sentinel bytes, so a stray write or a skipped -1 slot shows up anywhere.
"""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
import workloads
from pipeswift_amd import cache_ops, impl_utils, metadata
from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash, triton_reshape_and_cache_flash
from tests.conftest import raw

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32", torch.float8_e4m3fn: "fp8"}


def _run_case(case, dev, cache_dtype=None, k_scale=None, v_scale=None):
    print(f"append case: N={case.slot_mapping.shape[0]} H={case.num_heads} D={case.head_size} "
          f"cache={tuple(case.cache.shape)} {case.cache.dtype}", flush=True)
    qkv_d = case.qkv.to(dev)
    cache_d = case.cache.to(dev)
    ks = None if k_scale is None else torch.tensor([k_scale], dtype=torch.float32, device=dev)
    vs = None if v_scale is None else torch.tensor([v_scale], dtype=torch.float32, device=dev)
    reshape_and_cache_flash(case.key(qkv_d), case.value(qkv_d), cache_d[:, 0], cache_d[:, 1],
                            case.slot_mapping.to(dev), ks, vs)
    got = raw(cache_d)
    exp = raw(case.cache).copy()
    in_dt = DT[case.qkv.dtype]
    O.reshape_and_cache(raw(case.key()), raw(case.value()), exp[:, 0], exp[:, 1], case.slot_mapping.numpy(),
                        in_dt, DT[case.cache.dtype], k_scale, v_scale)
    return got, exp


def test_config1_bf16_append_whole_cache_bit_exact(dev):
    case = workloads.config1_append()
    assert case.num_valid == 486 and case.qkv.stride(0) == 6144
    got, exp = _run_case(case, dev)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_append_other_dtypes(dev, dtype):
    case = workloads.config1_append(seed=11, num_tokens=300, num_blocks=256, cache_dtype=dtype)
    case.qkv = case.qkv.to(dtype)
    got, exp = _run_case(case, dev)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("heads,head_size,block_size",
                         [(32, 128, 16), (12, 128, 32), (1, 64, 128), (4, 96, 12), (2, 40, 7), (64, 128, 16)])
def test_append_shapes(dev, heads, head_size, block_size):
    case = workloads.config1_append(seed=heads + head_size, num_tokens=257, num_blocks=97, block_size=block_size,
                                    heads=heads, head_size=head_size, q_size=head_size * heads)
    got, exp = _run_case(case, dev)
    assert np.array_equal(got, exp)


def test_append_prefill_sized_batch(dev):
    """4096+ tokens take the four-tokens-per-wave launch."""
    case = workloads.config1_append(seed=21, num_tokens=5000, num_blocks=1024)
    got, exp = _run_case(case, dev)
    assert np.array_equal(got, exp)


def test_append_split_caches_and_unaligned_rows(dev):
    """Separate K/V caches, a non-standard head stride (heads not adjacent)
    and an input row offset by one element (forces narrow vectors)."""
    g = torch.Generator().manual_seed(9)
    P, ps, H, D, N = 50, 16, 4, 64, 120
    big_k = workloads.sentinel((P, ps, H, D + 8), torch.bfloat16, 1)
    big_v = workloads.sentinel((P, ps, H, D + 8), torch.bfloat16, 2)
    qkv = torch.randn(N, 2 * H * D + 1, generator=g).to(torch.bfloat16)
    key = qkv[:, 1: 1 + H * D].view(N, H, D)
    value = qkv[:, 1 + H * D:].view(N, H, D)
    slots = torch.randperm(P * ps, generator=g)[:N].to(torch.int64)
    slots[5::11] = -1
    kd, vd = big_k.to(dev), big_v.to(dev)
    qd = qkv.to(dev)
    reshape_and_cache_flash(qd[:, 1: 1 + H * D].view(N, H, D), qd[:, 1 + H * D:].view(N, H, D),
                            kd[..., :D], vd[..., :D], slots.to(dev))
    ek, ev = raw(big_k).copy(), raw(big_v).copy()
    O.reshape_and_cache(raw(key), raw(value), ek[..., :D], ev[..., :D], slots.numpy())
    assert np.array_equal(raw(kd), ek) and np.array_equal(raw(vd), ev)


def test_append_strided_dim_takes_elementwise_path(dev):
    """A cache whose last dim is strided (dim stride 2) still matches."""
    g = torch.Generator().manual_seed(10)
    P, ps, H, D, N = 20, 8, 2, 16, 40
    base = workloads.sentinel((P, 2, ps, H, D, 2), torch.bfloat16, 3)
    qkv = torch.randn(N, 2 * H * D, generator=g).to(torch.bfloat16)
    slots = torch.randperm(P * ps, generator=g)[:N].to(torch.int64)
    bd = base.to(dev)
    qd = qkv.to(dev)
    reshape_and_cache_flash(qd[:, : H * D].view(N, H, D), qd[:, H * D:].view(N, H, D), bd[:, 0, ..., 0],
                            bd[:, 1, ..., 0], slots.to(dev))
    exp = raw(base).copy()
    O.reshape_and_cache(raw(qkv[:, : H * D].reshape(N, H, D)), raw(qkv[:, H * D:].reshape(N, H, D)),
                        exp[:, 0, ..., 0], exp[:, 1, ..., 0], slots.numpy())
    assert np.array_equal(raw(bd), exp)


def test_append_edge_slots(dev):
    """All -1, slots past the cache end and an empty batch leave the cache untouched."""
    case = workloads.config1_append(seed=12, num_tokens=64, num_blocks=32)
    case.slot_mapping[:] = -1
    case.slot_mapping[::3] = 32 * 16 + 5  # beyond the last slot: skipped, not written
    got, exp = _run_case(case, dev)
    assert np.array_equal(got, exp) and np.array_equal(got, raw(case.cache))
    cache_d = case.cache.to(dev)
    empty = torch.empty(0, 8, 128, dtype=torch.bfloat16, device=dev)
    reshape_and_cache_flash(empty, empty, cache_d[:, 0], cache_d[:, 1], torch.empty(0, dtype=torch.int64,
                                                                                     device=dev))
    assert np.array_equal(raw(cache_d), raw(case.cache))


def test_append_rejects_what_the_reference_asserts(dev):
    case = workloads.config1_append(seed=13, num_tokens=8, num_blocks=4)
    cache_d = case.cache.to(dev)
    qd = case.qkv.to(dev)
    with pytest.raises(AssertionError):
        reshape_and_cache_flash(case.key(qd), case.value(qd)[:, :4], cache_d[:, 0], cache_d[:, 1],
                                case.slot_mapping.to(dev))
    with pytest.raises(AssertionError):
        reshape_and_cache_flash(case.key(qd).float(), case.value(qd).float(), cache_d[:, 0], cache_d[:, 1],
                                case.slot_mapping.to(dev))
    with pytest.raises(AssertionError):  # int32 slots: the reference builds int64
        reshape_and_cache_flash(case.key(qd), case.value(qd), cache_d[:, 0], cache_d[:, 1],
                                case.slot_mapping.to(dev).int())
    assert triton_reshape_and_cache_flash is reshape_and_cache_flash


# --------------------------------------------------------------------------- #
# FP8
# --------------------------------------------------------------------------- #


def test_fp8_every_bf16_pattern_matches_golden_table(dev):
    """All 65536 bf16 bit patterns through the fused FP8 append at scale 1.0."""
    import os

    golden = np.fromfile(os.path.join(os.path.dirname(__file__), "golden", "e4m3_of_bf16.bin"), np.uint8)
    H, D = 4, 128
    N = 65536 // (H * D)
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).view(N, H, D)
    cache = torch.zeros(N, 2, 1, H, D, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    x = bits.to(dev)
    reshape_and_cache_flash(x, x, cache[:, 0], cache[:, 1], torch.arange(N, dtype=torch.int64, device=dev))
    got = raw(cache)
    # the table is torch's clamp (NaN kept: 0x7F|sign); the append stores the
    # reference's Triton clamp, which maps NaN to -448 (0xFE)
    exp = golden.copy()
    exp[np.isnan(O.bf16_to_f32(raw(bits).reshape(-1)))] = 0xFE
    assert np.array_equal(got[:, 0].reshape(-1), exp)
    assert np.array_equal(got[:, 1].reshape(-1), exp)


@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_scaled_boundaries_match_golden(dev, in_dtype):
    """The golden scaled set (ties, subnormals, saturation, +-0, +-inf) through
    the kernel: x / s in fp32, clamp, convert."""
    import os

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "e4m3_scaled.npz"))
    x, s, q = z["x"], z["scale"], z["q"]
    starts = np.flatnonzero(np.concatenate(([True], s[1:] != s[:-1])))
    ends = np.append(starts[1:], len(s))
    for a, b in zip(starts, ends):
        xs = torch.from_numpy(x[a:b].copy())
        if in_dtype != torch.float32:
            xs = xs.to(in_dtype)  # the input itself is rounded; the oracle sees the same rounded values
        n = xs.shape[0]
        cache = torch.zeros(n, 2, 1, 1, 1, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        xd = xs.view(n, 1, 1).to(dev)
        sc = torch.tensor([float(s[a])], dtype=torch.float32, device=dev)
        reshape_and_cache_flash(xd, xd, cache[:, 0], cache[:, 1], torch.arange(n, dtype=torch.int64, device=dev),
                                sc, sc)
        exp = O.quantize_e4m3(O.to_f32(raw(xs), DT[in_dtype]), float(s[a]), O.NAN_CLAMP_MIN)
        got = raw(cache)[:, 0].reshape(-1)
        assert np.array_equal(got, exp), f"scale {s[a]}"
        if in_dtype == torch.float32:
            assert np.array_equal(got, q[a:b])


@pytest.mark.parametrize("scale", [3.0, 7.77, 0.0123456789, 1e-3, 448.0 / 447.0, 2.5e-30, 3e29, 1e-39])
def test_fp8_every_bf16_pattern_at_scale(dev, scale):
    """All 65536 bf16 patterns at non-trivial scales: the reciprocal + FMA
    quotient must equal the IEEE fp32 quotient the oracle takes (1e-39 is a
    subnormal scale, which takes the plain division)."""
    H, D = 4, 128
    N = 65536 // (H * D)
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).view(N, H, D)
    cache = torch.zeros(N, 2, 1, H, D, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    x = bits.to(dev)
    sc = torch.tensor([scale], dtype=torch.float32, device=dev)
    reshape_and_cache_flash(x, x, cache[:, 0], cache[:, 1], torch.arange(N, dtype=torch.int64, device=dev), sc, sc)
    s32 = float(np.float32(scale))
    xf = O.bf16_to_f32(raw(bits).reshape(-1))
    exp = O.quantize_e4m3(xf, s32, O.NAN_CLAMP_MIN)
    assert np.array_equal(raw(cache)[:, 0].reshape(-1), exp)
    ref = raw((bits.float().reshape(-1) / torch.tensor(s32)).clamp(-448, 448).to(torch.float8_e4m3fn)).copy()
    ref[np.isnan(xf)] = 0xFE  # torch keeps NaN; the append stores the Triton clamp's -448
    assert np.array_equal(raw(cache)[:, 1].reshape(-1), ref)


def test_fp8_nan_policy(dev):
    """NaN inputs store -448 (0xFE) at every scale, as the reference's clamp
    tl.minimum(tl.maximum(x, -448), 448) does (Triton's minnum / maxnum);
    infinities saturate and -0 keeps its sign."""
    x = torch.tensor([float("nan"), -float("nan"), 1.0, float("inf"), -float("inf"), -0.0], dtype=torch.float32)
    n = x.shape[0]
    for scale in (None, 0.5, 1e-39):
        cache = torch.zeros(n, 2, 1, 1, 1, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        xd = x.view(n, 1, 1).to(dev)
        sc = None if scale is None else torch.tensor([scale], dtype=torch.float32, device=dev)
        reshape_and_cache_flash(xd, xd, cache[:, 0], cache[:, 1], torch.arange(n, dtype=torch.int64, device=dev),
                                sc, sc)
        want = [0xFE, 0xFE, 0x38 if scale is None else (0x40 if scale == 0.5 else 0x7E), 0x7E, 0xFE, 0x80]
        assert raw(cache)[:, 0].reshape(-1).tolist() == want, scale


@pytest.mark.parametrize("scale", [1.0, 7.77, -0.25, 1e-39])
def test_fp8_prefill_sized_every_bf16_pattern(dev, scale):
    """Every bf16 bit pattern (128 times each) through the prefill-sized FP8
    append: 4096 tokens of 8 x 128 K and V as column slices of 6144-wide qkv
    rows into 16-token pages in random order (the multi-token-per-wave
    scatter kernel), V at three times K's scale; whole cache against the
    oracle."""
    rng = np.random.default_rng(37)
    N, H, D, P, ps = 4096, 8, 128, 512, 16
    pats = np.tile(np.arange(65536, dtype=np.uint16), (2 * N * H * D) // 65536)
    rng.shuffle(pats)
    qkv = np.zeros((N, 6144), np.uint16)
    qkv[:, 4096:] = pats.reshape(N, 2 * H * D)
    qkv_t = torch.from_numpy(qkv.view(np.int16)).view(torch.bfloat16).to(dev)
    k, v = qkv_t[:, 4096:5120].view(N, H, D), qkv_t[:, 5120:].view(N, H, D)
    slots = torch.from_numpy(rng.permutation(P * ps)[:N].astype(np.int64))
    slots[::23] = -1
    cache = torch.zeros(P, 2, ps, H, D, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    ks = torch.tensor([scale], dtype=torch.float32, device=dev)
    vs = torch.tensor([scale * 3.0], dtype=torch.float32, device=dev)
    print(f"fp8 prefill-sized every bf16 pattern: N={N} scale={scale}", flush=True)
    reshape_and_cache_flash(k, v, cache[:, 0], cache[:, 1], slots.to(dev), ks, vs)
    exp = np.zeros((P, 2, ps, H, D), np.uint8)
    O.reshape_and_cache(raw(k), raw(v), exp[:, 0], exp[:, 1], slots.numpy(), "bf16", "fp8",
                        float(ks.cpu()), float(vs.cpu()))
    assert np.array_equal(raw(cache), exp)


def test_config2_fp8_decode_whole_cache(dev):
    """65536-block E4M3 cache (2 GiB fused; 64-bit offsets), scales from the
    amax kernel, whole-cache compare."""
    case = workloads.config2_fp8_decode()
    qd = case.qkv.to(dev)
    scales = cache_ops.compute_kv_scales(case.key(qd), case.value(qd))
    ks, ka = O.amax_scale(raw(case.key()), "bf16")
    vs, va = O.amax_scale(raw(case.value()), "bf16")
    assert scales.cpu().tolist() == [float(ks), float(vs)]
    cache_d = case.cache.to(dev)
    reshape_and_cache_flash(case.key(qd), case.value(qd), cache_d[:, 0], cache_d[:, 1], case.slot_mapping.to(dev),
                            scales[0:1], scales[1:2])
    got = raw(cache_d)
    exp = raw(case.cache).copy()
    O.reshape_and_cache(raw(case.key()), raw(case.value()), exp[:, 0], exp[:, 1], case.slot_mapping.numpy(),
                        "bf16", "fp8", ks, vs)
    assert np.array_equal(got, exp)


def test_fp8_prefill_append_whole_cache(dev):
    """The prefill-sized fused FP8 append (the bandwidth-bound shape the bench
    times): 8192 consecutive tokens in whole pages of config 2's 2 GiB cache,
    scales from the amax kernel, whole-cache compare against the oracle."""
    case = workloads.prefill_append(num_tokens=8192)
    print("fp8 prefill append: 8192 tokens, 65536 blocks", flush=True)
    qd = case.qkv.to(dev)
    scales = cache_ops.compute_kv_scales(case.key(qd), case.value(qd))
    ks, _ = O.amax_scale(raw(case.key()), "bf16")
    vs, _ = O.amax_scale(raw(case.value()), "bf16")
    assert scales.cpu().tolist() == [float(ks), float(vs)]
    cache_d = case.cache.to(dev)
    reshape_and_cache_flash(case.key(qd), case.value(qd), cache_d[:, 0], cache_d[:, 1], case.slot_mapping.to(dev),
                            scales[0:1], scales[1:2])
    got = raw(cache_d)
    exp = raw(case.cache).copy()
    O.reshape_and_cache(raw(case.key()), raw(case.value()), exp[:, 0], exp[:, 1], case.slot_mapping.numpy(),
                        "bf16", "fp8", ks, vs)
    assert np.array_equal(got, exp)


def test_bf16_prefill_append_whole_cache(dev):
    """The prefill-sized bf16 append (two resident workgroups per CU from 8192
    tokens): 8192 consecutive tokens in whole pages of a 4 GiB bf16 cache,
    whole-cache compare against the oracle."""
    case = workloads.prefill_append(num_tokens=8192, fp8=False)
    got, exp = _run_case(case, dev)
    assert np.array_equal(got, exp)


def test_append_offsets_beyond_2gib(dev):
    """A 4 GiB bf16 fused cache: blocks past byte 2^31 are addressed in 64 bits."""
    P, ps, H, D, N = 65536, 16, 8, 128, 256
    g = torch.Generator().manual_seed(19)
    cache = torch.zeros(P, 2, ps, H, D, dtype=torch.bfloat16, device=dev)
    blocks = torch.randperm(P - 40000, generator=g)[:N] + 40000  # byte offsets > 2^31
    offs = torch.randint(0, ps, (N,), generator=g)
    slots = (blocks * ps + offs).to(torch.int64)
    key = (torch.randn(N, H, D, generator=g) + 3).to(torch.bfloat16)
    value = (torch.randn(N, H, D, generator=g) - 3).to(torch.bfloat16)
    reshape_and_cache_flash(key.to(dev), value.to(dev), cache[:, 0], cache[:, 1], slots.to(dev))
    assert torch.equal(cache[blocks.to(dev), 0, offs.to(dev)].cpu().view(torch.int16), key.view(torch.int16))
    assert torch.equal(cache[blocks.to(dev), 1, offs.to(dev)].cpu().view(torch.int16), value.view(torch.int16))
    nz = int(torch.count_nonzero(cache.view(torch.int16)))
    assert nz == int(torch.count_nonzero(key.view(torch.int16))) + int(torch.count_nonzero(value.view(torch.int16)))


def test_amax_kernel_shapes(dev):
    g = torch.Generator().manual_seed(14)
    for shape, dtype in [((1000, 3, 7), torch.float32), ((5, 4096), torch.float16), ((1,), torch.bfloat16),
                         ((3000, 1024), torch.bfloat16)]:
        x = (torch.randn(shape, generator=g) * 50).to(dtype)
        if x.numel() > 10:
            x.view(-1)[7] = float("nan")
        s = cache_ops.compute_kv_scales(x.to(dev))
        es, ea = O.amax_scale(raw(x), DT[dtype])
        assert s.cpu().tolist() == [float(es)], (shape, dtype)
    z = cache_ops.compute_kv_scales(torch.zeros(64, 8, dtype=torch.bfloat16, device=dev))
    assert z.cpu().tolist() == [1.0]
    # strided rows (K and V slices of one qkv row) and repeated calls reuse the workspace
    case = workloads.config1_append(seed=15, num_tokens=777, num_blocks=64)
    qd = case.qkv.to(dev)
    for _ in range(3):
        s = cache_ops.compute_kv_scales(case.key(qd), case.value(qd))
    ks, _ = O.amax_scale(raw(case.key()), "bf16")
    vs, _ = O.amax_scale(raw(case.value()), "bf16")
    assert s.cpu().tolist() == [float(ks), float(vs)]


def test_kv_scales_replay_in_a_hip_graph(dev):
    """Both amax launches captured once and replayed over new data; every replay
    matches the oracle (no memset node, no workspace state carried over)."""
    from pipeswift_amd import fp8_kv

    fp8_kv.warmup(dev)
    g = torch.Generator().manual_seed(22)
    k_buf = torch.zeros(64, 8, 128, dtype=torch.bfloat16, device=dev)
    v_buf = torch.zeros(64, 8, 128, dtype=torch.bfloat16, device=dev)
    out = torch.zeros(2, dtype=torch.float32, device=dev)
    amax = torch.zeros(2, dtype=torch.float32, device=dev)
    cache_ops.compute_kv_scales(k_buf, v_buf, out=out, amax_out=amax)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            cache_ops.compute_kv_scales(k_buf, v_buf, out=out, amax_out=amax)
    torch.cuda.current_stream().wait_stream(s)
    for step in range(4):
        k = (torch.randn(64, 8, 128, generator=g) * (step + 1)).to(torch.bfloat16)
        v = (torch.randn(64, 8, 128, generator=g) * 0.1 / (step + 1)).to(torch.bfloat16)
        k_buf.copy_(k)
        v_buf.copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        ks, ka = O.amax_scale(raw(k), "bf16")
        vs, va = O.amax_scale(raw(v), "bf16")
        assert out.cpu().tolist() == [float(ks), float(vs)], f"replay {step}"
        assert amax.cpu().tolist() == [float(ka), float(va)], f"replay {step}"


# --------------------------------------------------------------------------- #
# impl_utils / metadata path and graph capture
# --------------------------------------------------------------------------- #


class _Seq:
    def __init__(self, seq_id, n_tokens, offset):
        self.seq_id = seq_id
        self.token_ids = list(range(n_tokens))
        self.offset = offset


def test_append_kv_cache_through_prepare_kv_info(dev):
    g = torch.Generator().manual_seed(16)
    L, P, ps, H, D = 3, 64, 16, 8, 128
    fused = workloads.sentinel((L, P, 2, ps, H, D), torch.bfloat16, 17)
    fd = fused.to(dev)
    kv_cache = [fd[:, :, 0], fd[:, :, 1]]
    seqs = [_Seq(0, 40, 0), _Seq(1, 70, 33), _Seq(2, 17, 16)]
    perm = torch.randperm(P - 1, generator=g) + 1
    table = {0: perm[0:3].tolist(), 1: perm[3:8].tolist(), 2: perm[8:10].tolist()}
    info = metadata.prepare_kv_info(seqs, table, ps, kv_cache, None, device=dev)
    n = info.slot_mapping.shape[0]
    key = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    value = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    impl_utils.append_kv_cache(key.to(dev), value.to(dev), info, layer_idx=1)
    exp = raw(fused).copy()
    slots = np.concatenate([O.slot_mapping(table[s.seq_id], s.offset, len(s.token_ids), ps) for s in seqs])
    assert np.array_equal(info.slot_mapping.cpu().numpy(), slots)
    O.reshape_and_cache(raw(key), raw(value), exp[1, :, 0], exp[1, :, 1], slots)
    assert np.array_equal(raw(fd), exp)


def test_append_replays_in_a_hip_graph(dev):
    """Captured append reading a static slot_mapping; every replay matches eager."""
    from pipeswift_amd import cudagraph

    P, ps, H, D, B = 128, 16, 8, 128, 32
    static = cudagraph.initialize_graph_kvcacheinfo(B, 8, device=dev)
    cache = torch.zeros(P, 2, ps, H, D, dtype=torch.bfloat16, device=dev)
    ref = cache.clone()
    key_buf = torch.zeros(B, H, D, dtype=torch.bfloat16, device=dev)
    val_buf = torch.zeros(B, H, D, dtype=torch.bfloat16, device=dev)
    # warm up outside capture, then capture on a side stream
    reshape_and_cache_flash(key_buf, val_buf, cache[:, 0], cache[:, 1], static.slot_mapping)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            reshape_and_cache_flash(key_buf, val_buf, cache[:, 0], cache[:, 1], static.slot_mapping)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(18)
    for step in range(5):
        bsz = 32 - 5 * step
        k = torch.randn(bsz, H, D, generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn(bsz, H, D, generator=g).to(torch.bfloat16).to(dev)
        slots = torch.randperm(P * ps, generator=g)[:bsz].to(torch.int64).to(dev)
        key_buf[:bsz].copy_(k)
        val_buf[:bsz].copy_(v)
        info = metadata.KVCacheInfo(page_table=torch.zeros(bsz, 8, dtype=torch.int32, device=dev),
                                    slot_mapping=slots, actual_lens_q=torch.ones(bsz, dtype=torch.int32, device=dev),
                                    actual_lens_kv=torch.ones(bsz, dtype=torch.int32, device=dev),
                                    cu_seqlens_q=torch.arange(bsz + 1, dtype=torch.int32, device=dev))
        cudagraph.set_graph_kvcacheinfo(static, info, B)
        graph.replay()
        reshape_and_cache_flash(k, v, ref[:, 0], ref[:, 1], slots)
        torch.cuda.synchronize()
        assert torch.equal(cache.view(torch.int16), ref.view(torch.int16)), f"replay {step}"
