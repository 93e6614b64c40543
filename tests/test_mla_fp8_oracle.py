"""Pins the oracle's tile-scaled FP8 MLA entry (oracle/kv_oracle.py,
quantize_mla_tiles / dequantize_mla_tiles / gather_mla_tiles) before it checks
the HIP kernels.

The reference names the scheme but has no code for it (it rejects FP8 for MLA,
pipeswift/utils/arguments.py:459-467), so the pins are independent of the
oracle's own formula: a hand-built entry whose bytes are known from the E4M3
code table, torch's CPU float8 conversion per tile (a library routine), the
scale recomputed in double precision from a Python max, the already-pinned
per-tensor quantizer, and the quantization error bound of a round trip.
"""

import struct

import numpy as np
import torch

from oracle import kv_oracle as O


def _bf16_bits(x) -> np.ndarray:
    return torch.as_tensor(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _e4m3_values(codes) -> np.ndarray:
    """float32 values of E4M3FN codes, decoded by torch."""
    return torch.tensor(np.asarray(codes, dtype=np.uint8)).view(torch.float8_e4m3fn).float().numpy()


def test_entry_size():
    assert O.mla_tile_entry_bytes(512, 64) == 656  # 512 fp8 + 4 fp32 scales + 64 bf16
    assert O.mla_tile_entry_bytes(128, 0) == 132


def test_known_answer_entry():
    """Tile j holds v * 2^(j-1) with v exactly representable in E4M3 and
    max |v| = 448, so s_j = 2^(j-1) and every code is the one v was taken from."""
    rng = np.random.default_rng(3)
    codes = np.empty((4, 128), dtype=np.uint8)
    for j in range(4):
        c = rng.choice(np.r_[0:0x7F, 0x80:0xFF], 128, replace=False).astype(np.uint8)  # no NaN codes
        c[rng.integers(128)] = 0x7E if j % 2 == 0 else 0xFE  # +-448 sets the tile max
        codes[j] = c
    v = _e4m3_values(codes)
    x = np.concatenate([v[j] * np.float32(2.0 ** (j - 1)) for j in range(4)])
    kv_c = _bf16_bits(x)[None]
    assert np.array_equal(O.bf16_to_f32(kv_c[0]), x)  # exact in bf16
    k_pe = np.arange(64, dtype=np.uint16)[None] * 1031
    want = bytearray(codes.reshape(-1).tobytes())
    want += b"".join(struct.pack("<f", 2.0 ** (j - 1)) for j in range(4))
    want += k_pe.astype("<u2").tobytes()
    got = O.quantize_mla_tiles(kv_c, k_pe)
    assert got.shape == (1, 656)
    assert got[0].tobytes() == bytes(want)
    back = O.dequantize_mla_tiles(got, 512, "f32").view(np.float32)
    assert np.array_equal(back[0, :512], x) and np.array_equal(back[0, 512:].view(np.uint32) >> 16, k_pe[0])


def test_tiles_match_torch_and_the_per_tensor_quantizer():
    g = torch.Generator().manual_seed(11)
    n, nope, rope = 24, 512, 64
    x = (torch.randn(n, nope, generator=g) * torch.logspace(-6, 6, n).unsqueeze(1)).to(torch.bfloat16)
    x[3, 17] = 900.0
    x[5, 130:140] = 0.0
    kv_c = x.view(torch.int16).numpy().view(np.uint16)
    k_pe = torch.randn(n, rope, generator=g).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ent = O.quantize_mla_tiles(kv_c, k_pe)
    xs = x.float()
    for t in range(n):
        for j in range(4):
            tile = xs[t, 128 * j: 128 * (j + 1)]
            amax = max(abs(float(v)) for v in tile)
            s = max(np.float32(amax / 448.0), np.float32(2.0 ** -126))  # double quotient, rounded once
            got_s = np.frombuffer(ent[t, 512 + 4 * j: 516 + 4 * j].tobytes(), dtype="<f4")[0]
            assert got_s == s, (t, j)
            ref = (tile / torch.tensor(s, dtype=torch.float32)).clamp(-448, 448).to(torch.float8_e4m3fn)
            assert np.array_equal(ent[t, 128 * j: 128 * (j + 1)], ref.view(torch.uint8).numpy()), (t, j)
            assert np.array_equal(ent[t, 128 * j: 128 * (j + 1)], O.quantize_e4m3(tile.numpy(), s))
    assert np.array_equal(ent[:, 528:].view(np.uint16), k_pe)


def test_round_trip_error_bound():
    """|x - q*s| <= s * max(2^-4 |x/s|, 2^-10): half an E4M3 step, normal or
    subnormal, in units of the tile scale."""
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(64, 512, generator=g) * 3).to(torch.bfloat16)
    x[:, ::97] *= 40
    kv_c = x.view(torch.int16).numpy().view(np.uint16)
    ent = O.quantize_mla_tiles(kv_c, np.zeros((64, 64), np.uint16))
    back = O.dequantize_mla_tiles(ent, 512, "f32").view(np.float32)[:, :512].astype(np.float64)
    xd = x.double().numpy()
    s = np.repeat(ent[:, 512:528].copy().view(np.float32), 128, axis=1).astype(np.float64)
    bound = s * np.maximum(2.0 ** -4 * np.abs(xd) / s, 2.0 ** -10) * (1 + 2.0 ** -16)
    assert np.all(np.abs(back - xd) <= bound)
    # and every tile's largest element lands on +-448 * s
    big = np.abs(back).reshape(64, 4, 128).max(axis=2)
    assert np.allclose(big, 448 * s[:, ::128], rtol=2.0 ** -20)


def test_zero_nan_and_infinite_tiles():
    x = np.zeros(512, np.float32)
    x[128:256] = np.linspace(-2, 2, 128, dtype=np.float32)
    x[140] = np.nan
    x[256:384] = 1.0
    x[300] = np.inf
    x[301] = -np.inf
    x[302] = -5.0
    x[384:] = 1e-37  # amax / 448 is below the 2^-126 floor
    kv_c = _bf16_bits(x)[None]
    kv_c[0, 140] = 0x7FC0  # a positive quiet NaN (torch's conversion gives 0xFFFF)
    kv_c[0, 141] = 0xFFC1  # a negative one
    ent = O.quantize_mla_tiles(kv_c, np.zeros((1, 64), np.uint16))[0]
    s = ent[512:528].copy().view(np.float32)
    assert s[0] == np.float32(2.0 ** -126) and not ent[:128].any()  # zero tile
    assert s[1] == np.float32(2.0 / 448)  # the NaN is ignored by the max
    assert ent[140] == 0x7F and ent[141] == 0xFF and ent[128] == 0xFE and ent[255] == 0x7E
    assert np.isinf(s[2])
    assert ent[300] == 0x7F and ent[301] == 0xFF  # +-inf / inf: NaN code, input's sign
    assert ent[302] == 0x80 and ent[256] == 0x00  # finite / inf: signed zero
    assert s[3] == np.float32(2.0 ** -126)
    xb = O.bf16_to_f32(kv_c[0, 384])
    assert ent[384] == O.quantize_e4m3(np.array([xb]), np.float32(2.0 ** -126))[0]
    back = O.dequantize_mla_tiles(ent[None], 512, "bf16")[0]
    assert back[140] == 0x7FC0 and back[0] == 0


def test_gather_of_entries_dequantizes_each_sequence():
    rng = np.random.default_rng(4)
    P, ps = 12, 4
    cache = rng.integers(0, 256, (P, ps, 656), dtype=np.uint8)
    cache[:, :, 512:528] = np.frombuffer(np.full(4, 0.5, np.float32).tobytes(), np.uint8)
    bt = np.array([[3, 7, 1], [11, 40, 2]], dtype=np.int32)  # 40 is out of range
    cu = np.array([0, 10, 19], dtype=np.int32)
    out = np.full((21, 576), 0xABCD, np.uint16)
    O.gather_mla_tiles(cache, bt, cu, 512, out=out)
    for b in range(2):
        for t in range(cu[b], cu[b + 1]):
            p = t - cu[b]
            blk = bt[b, p // ps]
            want = (np.zeros(576, np.uint16) if blk >= P
                    else O.dequantize_mla_tiles(cache[blk, p % ps][None], 512, "bf16")[0])
            assert np.array_equal(out[t], want), t
    assert np.all(out[19:] == 0xABCD)  # past the last sequence: untouched
    e = cache[3, 0]
    nope = O.bf16_to_f32(out[0, :512])
    ref = torch.tensor(e[:512]).view(torch.float8_e4m3fn).float() * 0.5
    assert np.array_equal(nope, ref.to(torch.bfloat16).float().numpy(), equal_nan=True)


def _rn32(q):
    """Round a Fraction to the nearest float32 (ties to even), normal range."""
    from fractions import Fraction

    if q == 0:
        return q
    if q < 0:
        return -_rn32(-q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    scaled = q / Fraction(2) ** (e - 23)  # in [2^23, 2^24)
    m, rem = divmod(scaled.numerator, scaled.denominator)
    twice = 2 * rem
    if twice > scaled.denominator or (twice == scaled.denominator and m % 2 == 1):
        m += 1
    return Fraction(m) * Fraction(2) ** (e - 23)


def test_tile_scale_division_method_is_correctly_rounded_for_every_bf16():
    """The append kernel divides amax by 448 as y = RN(amax * r), r = RN(1/448),
    then RN(y + (amax - y*448) * r) (two FMAs).  amax is always a bf16 value;
    for every positive normal bf16 from 2^-90 up this equals RN(amax / 448)."""
    from fractions import Fraction

    r = _rn32(Fraction(1, 448))
    assert float(r) == float(np.float32(1.0) / np.float32(448.0))
    bits = np.arange(0x0000, 0x7F80, dtype=np.uint32)
    vals = O.bf16_to_f32(bits.astype(np.uint16))
    checked = 0
    for v in vals[vals >= np.float32(2.0 ** -90)]:
        x = Fraction(float(v))
        y = _rn32(x * r)
        e = _rn32(x - y * 448)  # one FMA (the residual is exact; rounding it costs nothing)
        assert e == x - y * 448
        z = _rn32(y + e * r)
        assert z == _rn32(x / 448), float(v)
        checked += 1
    assert checked > 24000
