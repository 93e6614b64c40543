"""GPU parity of the MLA latent append and the block gather vs the CPU oracle."""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
import workloads
from pipeswift_amd import cache_ops, impl_utils, metadata
from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash, reshape_and_cache_flash_diffkv
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def _mla(case, dev, fp8_scale=None):
    n = case.slot_mapping.shape[0]
    print(f"mla case: N={n} cache={tuple(case.cache.shape)} fp8={fp8_scale is not None}", flush=True)
    latent_d = case.latent.to(dev)
    kv_c_d = case.kv_c.to(dev)
    if fp8_scale is None:
        cache_d = case.cache.to(dev)
        sc = None
    else:
        cache_d = torch.zeros(case.cache.shape, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        sc = torch.tensor([fp8_scale], dtype=torch.float32, device=dev)
    k_pe_d = case.k_pe(latent_d)
    assert k_pe_d.stride(0) == 2112
    reshape_and_cache_flash_diffkv(kv_c_d.unsqueeze(1), k_pe_d.unsqueeze(1), cache_d.unsqueeze(2),
                                   case.slot_mapping.to(dev), sc)
    if fp8_scale is None:
        exp = raw(case.cache).copy()
        O.concat_and_cache_mla(raw(case.kv_c), raw(case.k_pe()), exp, case.slot_mapping.numpy())
    else:
        exp = np.zeros(case.cache.shape, np.uint8)
        O.concat_and_cache_mla(raw(case.kv_c), raw(case.k_pe()), exp, case.slot_mapping.numpy(), "bf16", "fp8",
                               fp8_scale)
    return raw(cache_d), exp


@pytest.mark.parametrize("decode", [False, True])
def test_config4_mla_bf16(dev, decode):
    case = workloads.config4_mla(num_tokens=128 if decode else 4096, decode=decode)
    got, exp = _mla(case, dev)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("decode", [False, True])
def test_config4_mla_fp8(dev, decode):
    case = workloads.config4_mla(num_tokens=128 if decode else 4096, decode=decode)
    got, exp = _mla(case, dev, fp8_scale=0.0371)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("fp8", [False, True])
def test_mla_prefill_sized_append(dev, fp8):
    """A 16384-token MLA prefill (DeepSeek-V3 latent, pages of 64): the
    prefill-sized launch (two resident workgroups per CU for the bf16 copy),
    whole-cache compare."""
    case = workloads.config4_mla(num_tokens=16384)
    print(f"mla prefill append: 16384 tokens fp8={fp8}", flush=True)
    got, exp = _mla(case, dev, fp8_scale=0.0371 if fp8 else None)
    assert np.array_equal(got, exp)


def test_mla_fp8_append_wide_block_stride(dev):
    """Pages 16 MiB + 4 KiB apart: a block stride past 24 bits, so the packed
    FP8 append takes its 64-bit offset path (the narrow one needs every stride
    below 2^24 bytes); 1280 tokens, every slot of the 20 pages."""
    g = torch.Generator().manual_seed(35)
    P, ps, n = 20, 64, 1280
    pitch = (1 << 24) + 4096
    latent = torch.randn(n, 1536 + 576, generator=g).to(torch.bfloat16)
    ckv = torch.randn(n, 512, generator=g).to(torch.bfloat16)
    slots = torch.randperm(P * ps, generator=g).to(torch.int64)
    slots[::17] = -1
    base = torch.zeros(P, pitch, dtype=torch.uint8, device=dev)
    cache = base[:, : ps * 576].view(P, ps, 1, 576).view(torch.float8_e4m3fn)
    assert cache.stride(0) == pitch
    print(f"mla fp8 wide stride: N={n} pitch={pitch}", flush=True)
    ld = latent.to(dev)
    sc = torch.tensor([0.0371], dtype=torch.float32, device=dev)
    reshape_and_cache_flash_diffkv(ckv.to(dev).unsqueeze(1), ld[:, 2048:].unsqueeze(1), cache, slots.to(dev), sc)
    exp = np.zeros((P, ps, 576), np.uint8)
    O.concat_and_cache_mla(raw(ckv), raw(latent[:, 2048:]), exp, slots.numpy(), "bf16", "fp8", 0.0371)
    got = base.cpu().numpy()
    assert np.array_equal(got[:, : ps * 576].reshape(P, ps, 576), exp)
    assert not got[:, ps * 576 :].any()


@pytest.mark.parametrize("scale", [1.0, 0.0371, -0.5, 2.0 ** -90])
def test_mla_fp8_prefill_every_bf16_pattern(dev, scale):
    """Every bf16 bit pattern (NaNs, infinities, subnormals, signed zeros)
    through the packed FP8 MLA append (1152 tokens: the prefill-sized launch),
    k_pe a column slice of the latent, at scales on the quantizer's fast
    path, negative, and below its range (the IEEE division); whole cache
    against the oracle."""
    rng = np.random.default_rng(36)
    n, P, ps = 1152, 24, 64
    pats = np.tile(np.arange(65536, dtype=np.uint16), (n * 576) // 65536 + 1)[: n * 576]
    rng.shuffle(pats)
    rows = pats.reshape(n, 576)
    latent = np.zeros((n, 2112), np.uint16)
    latent[:, 2048:] = rows[:, 512:]
    latent_t = torch.from_numpy(latent.view(np.int16)).view(torch.bfloat16)
    ckv_t = torch.from_numpy(np.ascontiguousarray(rows[:, :512]).view(np.int16)).view(torch.bfloat16)
    slots = torch.from_numpy(rng.permutation(P * ps)[:n].astype(np.int64))
    slots[::19] = -1
    cache = torch.zeros(P, ps, 1, 576, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    sc = torch.tensor([scale], dtype=torch.float32, device=dev)
    print(f"mla fp8 every bf16 pattern: N={n} scale={scale}", flush=True)
    ld = latent_t.to(dev)
    reshape_and_cache_flash_diffkv(ckv_t.to(dev).unsqueeze(1), ld[:, 2048:].unsqueeze(1), cache, slots.to(dev), sc)
    exp = np.zeros((P, ps, 576), np.uint8)
    O.concat_and_cache_mla(raw(ckv_t), raw(latent_t[:, 2048:]), exp, slots.numpy(), "bf16", "fp8", scale)
    assert np.array_equal(raw(cache.cpu()).reshape(P, ps, 576), exp)


def test_mla_through_append_mla_kv_cache(dev):
    L, P, ps = 2, 300, 64
    mla = workloads.sentinel((L, P, ps, 576), torch.bfloat16, 31)
    md = mla.to(dev)
    g = torch.Generator().manual_seed(32)
    n = 200
    latent = torch.randn(n, 1536 + 576, generator=g).to(torch.bfloat16)
    ckv = torch.randn(n, 512, generator=g).to(torch.bfloat16)
    slots = torch.randperm(P * ps, generator=g)[:n].to(torch.int64)
    slots[::13] = -1
    info = metadata.KVCacheInfo(mla_cache_tensor=md, slot_mapping=slots.to(dev))
    ld = latent.to(dev)
    impl_utils.append_mla_kv_cache(ckv.to(dev), ld[:, 1536 + 512:], info, layer_idx=1)
    exp = raw(mla).copy()
    O.concat_and_cache_mla(raw(ckv), raw(latent[:, 2048:]), exp[1], slots.numpy())
    assert np.array_equal(raw(md), exp)


def test_mla_multi_head_flat_layout(dev):
    """H > 1: the reference writes all key elements then all value elements
    flat from the row start (reshape_and_cache.py:161-188)."""
    g = torch.Generator().manual_seed(33)
    n, H, Dk, Dv, P, ps = 50, 3, 16, 8, 20, 4
    key = torch.randn(n, H, Dk, generator=g).to(torch.bfloat16)
    value = torch.randn(n, H, Dv, generator=g).to(torch.bfloat16)
    cache = workloads.sentinel((P, ps, H, Dk + Dv), torch.bfloat16, 34)
    slots = torch.randperm(P * ps, generator=g)[:n].to(torch.int64)
    cd = cache.to(dev)
    reshape_and_cache_flash_diffkv(key.to(dev), value.to(dev), cd, slots.to(dev))
    exp = raw(cache).copy().reshape(P, ps, H * (Dk + Dv))
    O.concat_and_cache_mla(raw(key).reshape(n, -1), raw(value).reshape(n, -1), exp, slots.numpy())
    assert np.array_equal(raw(cd).reshape(P, ps, -1), exp)


# --------------------------------------------------------------------------- #
# chunked prefill append + gather (config 3)
# --------------------------------------------------------------------------- #


def test_config3_chunked_append_then_gather(dev):
    cc = workloads.config3_chunked()
    a = cc.append
    print(f"config3: chunks={cc.chunk.tolist()} prefix={cc.prefix.tolist()} T={int(cc.cu_seq_lens[-1])}",
          flush=True)
    qd = a.qkv.to(dev)
    cache_d = a.cache.to(dev)
    reshape_and_cache_flash(a.key(qd), a.value(qd), cache_d[:, 0], cache_d[:, 1], a.slot_mapping.to(dev))
    exp = raw(a.cache).copy()
    O.reshape_and_cache(raw(a.key()), raw(a.value()), exp[:, 0], exp[:, 1], a.slot_mapping.numpy())
    assert np.array_equal(raw(cache_d), exp)

    T = int(cc.cu_seq_lens[-1])
    out_k = torch.empty(T, a.num_heads, a.head_size, dtype=torch.bfloat16, device=dev)
    out_v = torch.empty_like(out_k)
    cache_ops.gather_cache(cache_d[:, 0], out_k, cc.block_table.to(dev), cc.cu_seq_lens.to(dev),
                           src_cache_v=cache_d[:, 1], dst_v=out_v)
    ek = O.gather_cache(exp[:, 0], cc.block_table.numpy(), cc.cu_seq_lens.numpy())
    ev = O.gather_cache(exp[:, 1], cc.block_table.numpy(), cc.cu_seq_lens.numpy())
    assert np.array_equal(raw(out_k), ek) and np.array_equal(raw(out_v), ev)
    # round trip: the newly appended chunk of every sequence reads back as its input rows
    cu = cc.cu_seq_lens.numpy()
    rows = []
    for b in range(len(cc.chunk)):
        rows.append(raw(out_k)[cu[b] + int(cc.prefix[b]): cu[b + 1]])
    assert np.array_equal(np.concatenate(rows), raw(a.key()))


def test_gather_fp8_dequant_seq_starts_and_bad_ids(dev):
    g = torch.Generator().manual_seed(35)
    P, ps, H, D = 64, 16, 4, 128
    cache = torch.randint(0, 256, (P, ps, H, D), generator=g, dtype=torch.uint8)
    cache[(cache & 0x7F) == 0x7F] = 0x11  # no NaN codes: NaN payloads are not pinned
    bt = torch.randperm(P, generator=g)[:24].to(torch.int32).view(3, 8)
    bt[0, 2] = 9999  # out of range -> zero rows
    bt[2, 0] = -5
    cu = torch.tensor([0, 40, 40, 100], dtype=torch.int32)
    starts = torch.tensor([16, 0, 3], dtype=torch.int32)
    cd = cache.to(dev).view(torch.float8_e4m3fn)
    scale = 0.0625 * 3
    for out_dtype, name in [(torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")]:
        out = torch.full((100, H, D), 7, dtype=out_dtype, device=dev)
        cache_ops.gather_cache(cd, out, bt.to(dev), cu.to(dev), seq_starts=starts.to(dev),
                               scale=torch.tensor([scale], dtype=torch.float32, device=dev))
        exp = O.gather_cache(cache.numpy(), bt.numpy(), cu.numpy(), seq_starts=starts.numpy(), cache_dtype="fp8",
                             out_dtype=name, scale=scale)
        assert np.array_equal(raw(out), exp), name
    raw_out = torch.zeros(100, H, D, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    cache_ops.gather_cache(cd, raw_out, bt.to(dev), cu.to(dev), seq_starts=starts.to(dev))
    exp = O.gather_cache(cache.numpy(), bt.numpy(), cu.numpy(), seq_starts=starts.numpy(), cache_dtype="fp8")
    assert np.array_equal(raw(raw_out), exp)


def test_gather_many_sequences_and_tail_untouched(dev):
    """300 sequences (binary search over cu_seq_lens), output longer than cu[-1]."""
    g = torch.Generator().manual_seed(36)
    P, ps, H, D = 2048, 16, 2, 64
    cache = workloads.sentinel((P, ps, H, D), torch.bfloat16, 37)
    lens = torch.randint(0, 90, (300,), generator=g)
    cu = torch.zeros(301, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    W = 6
    bt = torch.randint(0, P, (300, W), generator=g, dtype=torch.int32)
    T = int(cu[-1]) + 77
    cd = cache.to(dev)
    out = torch.full((T, H, D), 3, dtype=torch.bfloat16, device=dev)
    cache_ops.gather_cache(cd, out, bt.to(dev), cu.to(dev))
    exp = np.full((T, H, D), raw(torch.full((1,), 3, dtype=torch.bfloat16))[0], np.uint16)
    O.gather_cache(raw(cache), bt.numpy(), cu.numpy(), out=exp)
    assert np.array_equal(raw(out), exp)


@pytest.mark.parametrize("ps,H,D,with_starts", [(16, 8, 128, True), (12, 4, 128, True), (16, 2, 64, False),
                                                (5, 1, 64, True)])
def test_gather_many_sequences_kv_variants(dev, ps, H, D, with_starts):
    """Hundreds of sequences over 4096+ tokens (the four-tokens-per-wave launch
    and its sequence windows), K and V in one launch, page-aligned and
    unaligned seq_starts, power-of-two and other block sizes, 2 KiB rows."""
    g = torch.Generator().manual_seed(38 + ps + H)
    P = 4096
    kc = workloads.sentinel((P, ps, H, D), torch.bfloat16, 39)
    vc = workloads.sentinel((P, ps, H, D), torch.bfloat16, 40)
    B = 230
    lens = torch.randint(0, 60, (B,), generator=g)
    lens[::17] = 0
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    starts = torch.randint(0, 3 * ps, (B,), generator=g).to(torch.int32) if with_starts else None
    W = (60 + 3 * ps) // ps + 2
    bt = torch.randint(0, P, (B, W), generator=g, dtype=torch.int32)
    bt[3, 1] = P + 5  # out of range -> zero rows
    T = int(cu[-1]) + 9
    assert T >= 4096
    out_k = torch.full((T, H, D), 3, dtype=torch.bfloat16, device=dev)
    out_v = torch.full((T, H, D), 3, dtype=torch.bfloat16, device=dev)
    cache_ops.gather_cache(kc.to(dev), out_k, bt.to(dev), cu.to(dev), src_cache_v=vc.to(dev), dst_v=out_v,
                           seq_starts=None if starts is None else starts.to(dev))
    fill = raw(torch.full((1,), 3, dtype=torch.bfloat16))[0]
    for cache, out in ((kc, out_k), (vc, out_v)):
        exp = np.full((T, H, D), fill, np.uint16)
        O.gather_cache(raw(cache), bt.numpy(), cu.numpy(), seq_starts=None if starts is None else starts.numpy(),
                       out=exp)
        assert np.array_equal(raw(out), exp)


@pytest.mark.parametrize("ps,H,D,dequant,pad", [(16, 4, 128, False, 0), (16, 8, 128, False, 64),
                                                (16, 16, 128, False, 0), (24, 4, 128, False, 0),
                                                (16, 4, 128, True, 0), (32, 8, 128, True, 128)])
def test_gather_large_mixed_sequences(dev, ps, H, D, dequant, pad):
    """Gathers of 4096+ tokens (the multi-token-per-wave launches) with rows of
    64, 128 or 256 16-byte vectors: long and short sequences so a wave's
    tokens start inside sequences and straddle their ends, more than 64
    sequences, seq_starts, bad block ids, padded output rows, fp8
    dequantization, output rows past the batch untouched."""
    g = torch.Generator().manual_seed(50 + ps + H + int(dequant))
    P, B = 4096, 90
    row = H * D
    lens = torch.randint(0, 40, (B,), generator=g)
    lens[::11] = torch.randint(300, 1500, (len(lens[::11]),), generator=g)
    lens[5] = 0
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    starts = torch.randint(0, 2 * ps, (B,), generator=g).to(torch.int32)
    W = (int(lens.max()) + 2 * ps) // ps + 1
    bt = torch.randint(0, P, (B, W), generator=g, dtype=torch.int32)
    bt[0, 1] = P + 3  # out of range -> zero rows
    bt[11, 0] = -2
    T = int(cu[-1]) + 21
    assert T >= 4096
    if dequant:
        caches = [torch.randint(0, 256, (P, ps, H, D), generator=g, dtype=torch.uint8) for _ in range(2)]
        for c in caches:
            c[(c & 0x7F) == 0x7F] = 0x21  # no NaN codes: NaN payloads are not pinned
        src = [c.to(dev).view(torch.float8_e4m3fn) for c in caches]
        out_dt, scale = torch.bfloat16, 0.375
    else:
        caches = [workloads.sentinel((P, ps, H, D), torch.bfloat16, 51 + i) for i in range(2)]
        src = [c.to(dev) for c in caches]
        out_dt, scale = torch.bfloat16, None
    print(f"large gather: ps={ps} H={H} D={D} dequant={dequant} pad={pad} T={T}", flush=True)
    full = [torch.full((T, row + pad), 3, dtype=out_dt, device=dev) for _ in range(2)]
    outs = [f[:, :row].view(T, H, D) for f in full]
    cache_ops.gather_cache(src[0], outs[0], bt.to(dev), cu.to(dev), seq_starts=starts.to(dev),
                           scale=None if scale is None else torch.tensor([scale], dtype=torch.float32, device=dev),
                           src_cache_v=src[1], dst_v=outs[1])
    fill = raw(torch.full((1,), 3, dtype=out_dt))[0]
    for cache, f in zip(caches, full):
        exp = np.full((T, row + pad), fill, np.uint16)
        body = exp[:, :row].reshape(T, H, D)
        if dequant:
            got = O.gather_cache(cache.numpy(), bt.numpy(), cu.numpy(), seq_starts=starts.numpy(),
                                 cache_dtype="fp8", out_dtype="bf16", scale=scale, out=body.copy())
        else:
            got = O.gather_cache(raw(cache), bt.numpy(), cu.numpy(), seq_starts=starts.numpy(), out=body.copy())
        exp[:, :row] = got.reshape(T, row)
        assert np.array_equal(raw(f), exp)


def test_chunked_prefill_16k_append_then_gather(dev):
    """Config 3's geometry with a 16384-token chunk over 6 sequences: the
    prefill-sized append launch (two resident workgroups per CU for the bf16
    copy), then the gather, against the oracle and as a round trip."""
    cc = workloads.config3_chunked(batched_tokens=16384)
    a = cc.append
    print(f"chunked 16k: chunks={cc.chunk.tolist()} T={int(cc.cu_seq_lens[-1])}", flush=True)
    qd = a.qkv.to(dev)
    cache_d = a.cache.to(dev)
    reshape_and_cache_flash(a.key(qd), a.value(qd), cache_d[:, 0], cache_d[:, 1], a.slot_mapping.to(dev))
    exp = raw(a.cache).copy()
    O.reshape_and_cache(raw(a.key()), raw(a.value()), exp[:, 0], exp[:, 1], a.slot_mapping.numpy())
    assert np.array_equal(raw(cache_d), exp)
    T = int(cc.cu_seq_lens[-1])
    out_k = torch.empty(T, a.num_heads, a.head_size, dtype=torch.bfloat16, device=dev)
    out_v = torch.empty_like(out_k)
    cache_ops.gather_cache(cache_d[:, 0], out_k, cc.block_table.to(dev), cc.cu_seq_lens.to(dev),
                           src_cache_v=cache_d[:, 1], dst_v=out_v)
    cu = cc.cu_seq_lens.numpy()
    rows_k = np.concatenate([raw(out_k)[cu[b] + int(cc.prefix[b]): cu[b + 1]] for b in range(len(cc.chunk))])
    rows_v = np.concatenate([raw(out_v)[cu[b] + int(cc.prefix[b]): cu[b + 1]] for b in range(len(cc.chunk))])
    assert np.array_equal(rows_k, raw(a.key())) and np.array_equal(rows_v, raw(a.value()))


def test_config3_block_size_128_append_then_gather(dev):
    """Config 3's sensitivity run: the same chunked prefill at 128-token pages
    (4096 blocks, the same slot capacity), append then gather, against the
    oracle and as a round trip."""
    cc = workloads.config3_chunked(block_size=128, num_blocks=4096)
    a = cc.append
    print(f"config3 ps=128: chunks={cc.chunk.tolist()} prefix={cc.prefix.tolist()} T={int(cc.cu_seq_lens[-1])}",
          flush=True)
    qd = a.qkv.to(dev)
    cache_d = a.cache.to(dev)
    reshape_and_cache_flash(a.key(qd), a.value(qd), cache_d[:, 0], cache_d[:, 1], a.slot_mapping.to(dev))
    exp = raw(a.cache).copy()
    O.reshape_and_cache(raw(a.key()), raw(a.value()), exp[:, 0], exp[:, 1], a.slot_mapping.numpy())
    assert np.array_equal(raw(cache_d), exp)
    T = int(cc.cu_seq_lens[-1])
    out_k = torch.empty(T, a.num_heads, a.head_size, dtype=torch.bfloat16, device=dev)
    out_v = torch.empty_like(out_k)
    cache_ops.gather_cache(cache_d[:, 0], out_k, cc.block_table.to(dev), cc.cu_seq_lens.to(dev),
                           src_cache_v=cache_d[:, 1], dst_v=out_v)
    assert np.array_equal(raw(out_k), O.gather_cache(exp[:, 0], cc.block_table.numpy(), cc.cu_seq_lens.numpy()))
    assert np.array_equal(raw(out_v), O.gather_cache(exp[:, 1], cc.block_table.numpy(), cc.cu_seq_lens.numpy()))
    cu = cc.cu_seq_lens.numpy()
    rows = [raw(out_v)[cu[b] + int(cc.prefix[b]): cu[b + 1]] for b in range(len(cc.chunk))]
    assert np.array_equal(np.concatenate(rows), raw(a.value()))
