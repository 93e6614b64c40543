"""Pins the CPU oracle (oracle/kv_oracle.py) before it is trusted as the checker.

Each check is independent of the oracle's own formula: torch's CPU dtype
conversions (library routines), torch index_put_/index_select on the same
strided layouts, literal hand-computed tiny caches, invariants (untouched
slots, round trips) and brute force.
"""

import os

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.conftest import raw

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# --------------------------------------------------------------------------- #
# element conversions
# --------------------------------------------------------------------------- #


def test_e4m3_of_every_bf16_matches_golden_and_torch():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mine = O.quantize_e4m3(O.bf16_to_f32(bits), 1.0)
    golden = np.fromfile(os.path.join(GOLDEN, "e4m3_of_bf16.bin"), dtype=np.uint8)
    assert golden.shape == (65536,)
    assert np.array_equal(mine, golden)
    t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    ref = t.float().clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_unsaturated_e4m3_conversion_matches_torch_everywhere():
    """The raw conversion (no clamp): overflow and inf go to the NaN code."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    ref = t.float().to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.e4m3fn_from_f32(O.bf16_to_f32(bits)), ref)
    x = np.random.default_rng(3).standard_normal(200000).astype(np.float32) * np.float32(100)
    x = np.concatenate([x, np.float32(2.0) ** np.arange(-20, 12, dtype=np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.e4m3fn_from_f32(x), ref)


def test_scaled_quantize_matches_golden():
    z = np.load(os.path.join(GOLDEN, "e4m3_scaled.npz"))
    got = np.concatenate([O.quantize_e4m3(z["x"][i:i + 1], float(z["scale"][i])) for i in range(0, 300)])
    assert np.array_equal(got, z["q"][:300])
    # vectorised over runs of equal scale
    s = z["scale"]
    starts = np.flatnonzero(np.concatenate(([True], s[1:] != s[:-1])))
    ends = np.append(starts[1:], len(s))
    for a, b in zip(starts, ends):
        assert np.array_equal(O.quantize_e4m3(z["x"][a:b], float(s[a])), z["q"][a:b])


def test_e4m3_known_codes():
    cases = [(0.0, 0x00), (-0.0, 0x80), (448.0, 0x7E), (-448.0, 0xFE), (2.0 ** -9, 0x01), (2.0 ** -6, 0x08),
             (1.0, 0x38), (1.5, 0x3C), (1.0625, 0x38), (1.1875, 0x3A), (464.0, 0x7E), (500.0, 0x7E),
             (np.inf, 0x7E), (-np.inf, 0xFE), (2.0 ** -10, 0x00), (3 * 2.0 ** -10, 0x02)]
    for x, code in cases:
        assert O.quantize_e4m3(np.array([x], np.float32), 1.0)[0] == code, x
    assert O.quantize_e4m3(np.array([np.nan], np.float32), 1.0)[0] == 0x7F
    assert O.quantize_e4m3(np.array([-np.nan], np.float32), 1.0)[0] == 0xFF
    for v in (np.nan, -np.nan):
        assert O.quantize_e4m3(np.array([v], np.float32), 1.0, O.NAN_CLAMP_MIN)[0] == 0xFE


def test_append_nan_policy_is_the_references_triton_clamp():
    """The append's clamp is Triton's tl.minimum(tl.maximum(x, -448), 448)
    (reshape_and_cache.py:70-75) with the default PropagateNan.NONE, i.e. LLVM
    maxnum / minnum, which return the non-NaN operand (Triton 3.6:
    language/core.py:2506,2528, semantic.py:380-381).  numpy's fmax / fmin have
    those semantics: evaluating the reference's expression with them and
    converting with torch gives the oracle's NAN_CLAMP_MIN bytes for every bf16
    pattern, at scale 1 and at a scale != 1 (where x / s is clamped)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = O.bf16_to_f32(bits)
    for scale in (1.0, 0.37):
        with np.errstate(invalid="ignore", over="ignore"):
            y = (x / np.float32(scale)).astype(np.float32)
        clamped = np.fmin(np.fmax(y, np.float32(-448.0)), np.float32(448.0))
        assert not np.isnan(clamped).any()
        ref = torch.from_numpy(clamped).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(O.quantize_e4m3(x, scale, O.NAN_CLAMP_MIN), ref)
    # the append oracle uses it
    cache = np.zeros((2, 2, 1, 3), np.uint8)
    kv = np.array([[[0x7FC0, 0xFFC0, 0x3F80]]], np.uint16)
    O.reshape_and_cache(kv, kv, cache[:, 0], cache[:, 1], np.array([1]), "bf16", "fp8")
    assert cache[1, 0, 0].tolist() == [0xFE, 0xFE, 0x38]


def test_e4m3_decode_matches_torch():
    b = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(O.e4m3fn_to_f32(b), ref, equal_nan=True)
    assert np.isnan(O.e4m3fn_to_f32(np.array([0x7F, 0xFF], np.uint8))).all()


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(1).standard_normal(300000).astype(np.float32) * np.float32(1e4)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.00390625,
                                     1.01171875], np.float32)])
    ref = raw(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(O.bf16_from_f32(x), ref)
    # NaN payloads are not pinned (torch's vector path emits 0xFFFF, scalar 0x7FC0); the class is
    out = O.bf16_from_f32(np.array([np.nan], np.float32))
    assert np.isnan(O.bf16_to_f32(out)).all()


def test_dequantize_matches_torch():
    q = np.arange(256, dtype=np.uint8)
    q = q[(q & 0x7F) != 0x7F]
    for s in (1.0, 0.37, 5.5):
        ref = raw((torch.from_numpy(q).view(torch.float8_e4m3fn).float() * torch.tensor(s, dtype=torch.float32))
                  .to(torch.bfloat16))
        assert np.array_equal(O.dequantize_e4m3(q, s, "bf16"), ref)


# --------------------------------------------------------------------------- #
# append
# --------------------------------------------------------------------------- #


def test_append_literal_tiny_case():
    """P=2 blocks of ps=2 slots, H=1, D=2; every expected byte written out."""
    key = np.array([[[1, 2]], [[3, 4]], [[5, 6]]], np.uint16)
    value = key + 100
    fused = np.full((2, 2, 2, 1, 2), 9, np.uint16)  # [P, K/V, ps, H, D]
    O.reshape_and_cache(key, value, fused[:, 0], fused[:, 1], np.array([3, -1, 0]))
    exp = np.array([
        [[[[5, 6]], [[9, 9]]], [[[105, 106]], [[9, 9]]]],
        [[[[9, 9]], [[1, 2]]], [[[9, 9]], [[101, 102]]]],
    ], np.uint16)
    assert np.array_equal(fused, exp)


def test_append_matches_torch_index_put_on_fused_layout():
    g = torch.Generator().manual_seed(5)
    P, ps, H, D, N = 32, 16, 4, 64, 200
    fused = torch.randint(-30000, 30000, (P, 2, ps, H, D), generator=g, dtype=torch.int16).view(torch.bfloat16)
    qkv = torch.randn(N, 6 * H * D, generator=g).to(torch.bfloat16)
    key = qkv[:, 2 * H * D: 3 * H * D].view(N, H, D)
    value = qkv[:, 3 * H * D: 4 * H * D].view(N, H, D)
    slots = torch.randperm(P * ps, generator=g)[:N]
    slots[::9] = -1
    ref = fused.clone()
    valid = slots >= 0
    s = slots[valid]
    ref[:, 0].index_put_((s // ps, s % ps), key[valid])
    ref[:, 1].index_put_((s // ps, s % ps), value[valid])
    got = raw(fused).copy()
    O.reshape_and_cache(raw(key), raw(value), got[:, 0], got[:, 1], slots.numpy())
    assert np.array_equal(got, raw(ref))


def test_append_fp8_matches_torch():
    g = torch.Generator().manual_seed(6)
    P, ps, H, D, N = 16, 8, 2, 32, 60
    cache = torch.zeros(P, 2, ps, H, D, dtype=torch.uint8)
    key = (torch.randn(N, H, D, generator=g) * 100).to(torch.bfloat16)
    value = (torch.randn(N, H, D, generator=g) * 3).to(torch.bfloat16)
    slots = torch.randperm(P * ps, generator=g)[:N]
    ks, vs = 0.73, 1.0
    ref = cache.clone()
    ref[:, 0][slots // ps, slots % ps] = (key.float() / ks).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    ref[:, 1][slots // ps, slots % ps] = (value.float() / vs).clamp(-448, 448).to(torch.float8_e4m3fn).view(
        torch.uint8)
    got = cache.numpy().copy()
    O.reshape_and_cache(raw(key), raw(value), got[:, 0], got[:, 1], slots.numpy(), "bf16", "fp8", ks, vs)
    assert np.array_equal(got, ref.numpy())


def test_append_skips_out_of_range_and_negative_slots():
    cache = np.zeros((2, 2, 4, 1, 2), np.uint16)
    key = np.ones((3, 1, 2), np.uint16)
    O.reshape_and_cache(key, key, cache[:, 0], cache[:, 1], np.array([-1, 8, 1_000_000]))
    assert not cache.any()


# --------------------------------------------------------------------------- #
# MLA, gather, copy_blocks
# --------------------------------------------------------------------------- #


def test_mla_literal_tiny_case():
    kv_c = np.array([[1, 2, 3], [4, 5, 6]], np.uint16)
    k_pe = np.array([[7], [8]], np.uint16)
    cache = np.zeros((2, 2, 4), np.uint16)
    O.concat_and_cache_mla(kv_c, k_pe, cache, np.array([2, 1]))
    exp = np.zeros((2, 2, 4), np.uint16)
    exp[1, 0] = [1, 2, 3, 7]
    exp[0, 1] = [4, 5, 6, 8]
    assert np.array_equal(cache, exp)


def test_gather_literal_and_round_trip():
    ps = 2
    cache = np.arange(4 * ps * 3, dtype=np.uint16).reshape(4, ps, 3)
    bt = np.array([[3, 1, 0], [2, 0, 0]], np.int32)
    cu = np.array([0, 5, 7], np.int32)
    out = O.gather_cache(cache, bt, cu)
    exp = np.stack([cache[3, 0], cache[3, 1], cache[1, 0], cache[1, 1], cache[0, 0], cache[2, 0], cache[2, 1]])
    assert np.array_equal(out, exp)
    # seq_starts offsets positions; ids out of range give zeros
    out2 = O.gather_cache(cache, np.array([[3, 99]], np.int32), np.array([0, 3], np.int32),
                          seq_starts=np.array([1], np.int32))
    assert np.array_equal(out2, np.stack([cache[3, 1], np.zeros(3, np.uint16), np.zeros(3, np.uint16)]))


def test_gather_inverts_append():
    rng = np.random.default_rng(11)
    P, ps, H, D = 40, 16, 2, 8
    lens = [37, 0, 64, 5]
    pages = [-(-n // ps) for n in lens]
    perm = rng.permutation(P)
    bt = np.zeros((len(lens), max(pages)), np.int32)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off: off + n]
        off += n
    key = rng.integers(0, 65535, (sum(lens), H, D), dtype=np.uint16)
    slots = np.concatenate([bt[b, np.arange(n) // ps].astype(np.int64) * ps + np.arange(n) % ps
                            for b, n in enumerate(lens)])
    cache = np.zeros((P, 2, ps, H, D), np.uint16)
    O.reshape_and_cache(key, key, cache[:, 0], cache[:, 1], slots)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    assert np.array_equal(O.gather_cache(cache[:, 0], bt, cu), key)


def test_gather_matches_torch_index_select():
    g = torch.Generator().manual_seed(2)
    P, ps, H, D = 30, 4, 2, 8
    cache = torch.randint(0, 60000, (P, ps, H, D), generator=g, dtype=torch.int32).to(torch.int16)
    lens = [9, 12, 1]
    bt = torch.stack([torch.randperm(P, generator=g)[:4] for _ in lens]).to(torch.int32)
    cu = torch.tensor([0, 9, 21, 22], dtype=torch.int32)
    ref = torch.cat([cache.index_select(0, bt[b].long()).reshape(-1, H, D)[: lens[b]] for b in range(3)])
    got = O.gather_cache(cache.numpy().view(np.uint16), bt.numpy(), cu.numpy())
    assert np.array_equal(got, ref.numpy().view(np.uint16))


def test_copy_blocks_matches_clone_and_is_idempotent():
    g = torch.Generator().manual_seed(4)
    L, P = 3, 20
    stack = torch.randint(0, 1000, (L, P, 2, 4), generator=g, dtype=torch.int32)
    perm = torch.randperm(P, generator=g)
    m = torch.stack([perm[:6], perm[6:12]], 1)
    ref = stack.clone()
    ref[:, m[:, 1]] = stack[:, m[:, 0]].clone()
    got = stack.numpy().copy()
    O.copy_blocks(got, m.numpy())
    assert np.array_equal(got, ref.numpy())
    O.copy_blocks(got, m.numpy())
    assert np.array_equal(got, ref.numpy())
    O.validate_block_mapping(m.numpy(), P)
    with pytest.raises(AssertionError):
        O.validate_block_mapping(np.array([[1, 2], [2, 3]]), P)
    with pytest.raises(AssertionError):
        O.validate_block_mapping(np.array([[1, 2], [4, 2]]), P)
    with pytest.raises(AssertionError):
        O.validate_block_mapping(np.array([[1, P]]), P)


def test_amax_scale_matches_torch():
    x = (torch.randn(64, 256, generator=torch.Generator().manual_seed(8)) * 9).to(torch.bfloat16)
    x[3, 7] = float("nan")
    s, a = O.amax_scale(raw(x), "bf16")
    xf = x.float()
    amax = xf[~xf.isnan()].abs().max()
    assert a == amax.item()
    assert s == (amax / torch.tensor(448.0)).item()
    s0, a0 = O.amax_scale(np.zeros(10, np.uint16), "bf16")
    assert s0 == 1.0 and a0 == 0.0


# --------------------------------------------------------------------------- #
# transport helpers and slot mapping
# --------------------------------------------------------------------------- #


def _brute_runs(src, dst):
    pairs = sorted(zip(src, dst), key=lambda p: p[0])
    runs = []
    for s, d in pairs:
        if runs and runs[-1][0] + runs[-1][2] == s and runs[-1][1] + runs[-1][2] == d:
            runs[-1][2] += 1
        else:
            runs.append([s, d, 1])
    return runs


@pytest.mark.parametrize("seed", range(20))
def test_coalesce_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 60))
    src = rng.permutation(100)[:n]
    if seed % 3 == 0:
        src = np.sort(src)
    dst = src + 7 if seed % 2 == 0 else rng.permutation(100)[:n]
    s, d, ln = O.coalesce(src, dst)
    assert [list(map(int, r)) for r in zip(s, d, ln)] == _brute_runs(src.tolist(), dst.tolist())


def _brute_slots(pt, offset, ntok, ps, dcp, rank, il):
    """Per-position restatement written from the DCP ownership rule directly."""
    out = []
    for pos in range(offset, ntok):
        owner = (pos // il) % dcp
        if owner != rank:
            out.append(-1)
            continue
        # local index = number of earlier positions this rank owns
        local = sum(1 for q in range(pos) if (q // il) % dcp == rank)
        phys = ps // dcp
        out.append(pt[pos // ps] * phys + local % phys)
    return out


@pytest.mark.parametrize("dcp,il", [(1, 1), (2, 1), (2, 4), (4, 2), (4, 4)])
def test_slot_mapping_matches_brute_force(dcp, il):
    rng = np.random.default_rng(dcp * 10 + il)
    ps = 16
    pt = rng.permutation(50)[:12].tolist()
    for rank in range(dcp):
        for offset, ntok in [(0, 150), (37, 120), (0, 1), (64, 65)]:
            got = O.slot_mapping(pt, offset, ntok, ps, dcp, rank, il)
            assert got == _brute_slots(pt, offset, ntok, ps, dcp, rank, il)
            # dcp_kv_len counts the rank's positions in [0, ntok)
            assert O.dcp_kv_len(ntok, dcp, rank, il) == sum(1 for q in range(ntok) if (q // il) % dcp == rank)
