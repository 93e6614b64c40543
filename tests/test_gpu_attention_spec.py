"""GPU parity of the paged attention reader with several query tokens per
sequence (speculative / multi-token decode: psk_paged_decode_attention with
q_len > 1, ragged cu_seqlens_q, causal with FA's bottom-right alignment).

The query tokens of a sequence and the query heads of a kv head share the 16
rows of one MFMA tile, so the arithmetic per row is that of one-token decode
and so are the tolerances (see test_gpu_attention.py):
  * fp32 output: |got - oracle| <= 3e-4 * max|V * vd| + 1e-4 * |oracle|
  * bf16 output: the same plus one bf16 rounding (2^-8 relative)
  * lse:         |got - oracle| <= 5e-4 + 1e-5 * |oracle|
The oracle (oracle/kv_oracle.py: paged_decode_attention) runs in float64 and is
pinned against torch SDPA under torch's lower-right causal mask.
"""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd import attention
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def _fp8(shape, std, gen):
    return (torch.randn(shape, generator=gen) * std).to(torch.float8_e4m3fn)


def _check(got, exp, vmax, bf16):
    got = got.float().cpu().numpy().astype(np.float64)
    tol = 3e-4 * vmax + (2.0 ** -8 + 1e-4 if bf16 else 1e-4) * np.abs(exp)
    err = np.abs(got - exp)
    assert (err <= tol).all(), f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


def _spec_case(dev, seed, lens, counts, Hq, Hkv, ps, q_len, causal, q_dtype="bf16", out_dtype=torch.float32,
               descales=True, num_splits=0, ragged=True, P=None):
    """counts[b] query tokens for sequence b (all q_len when not ragged, and
    then cu_seqlens_q is left out)."""
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    need = sum(-(-x // ps) for x in lens) + 8
    P = P or max(64, need)
    fused = torch.zeros(P, 2, ps, Hkv, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, Hkv, 128), 2.0, g)
    fused[:, 1] = _fp8((P, ps, Hkv, 128), 2.0, g)
    W = max(1, max(-(-x // ps) for x in lens))
    bt = torch.stack([torch.randperm(P, generator=g)[:W] for _ in range(B)]).to(torch.int32)
    counts = list(counts) if ragged else [q_len] * B
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    TQ = int(cu[-1])
    qb = (torch.randn(TQ, Hq, 128, generator=g) * 3).to(torch.bfloat16)
    q = qb.clamp(-448, 448).to(torch.float8_e4m3fn) if q_dtype == "fp8" else qb
    rng = np.random.default_rng(seed)
    ds = [torch.from_numpy(rng.uniform(0.5, 2.0, (B, Hkv)).astype(np.float32)) for _ in range(3)] if descales \
        else [None] * 3
    fd = fused.to(dev)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    # rows of out that the call writes are all of them; fill with a sentinel
    out = torch.full((TQ, Hq, 128), 7.0, dtype=out_dtype, device=dev)
    print(f"spec case seed={seed} B={B} Hq={Hq} Hkv={Hkv} ps={ps} q_len={q_len} causal={causal} "
          f"ragged={ragged} splits={num_splits}", flush=True)
    got, lse = attention.paged_decode_attention(
        q.to(dev), fd[:, 0], fd[:, 1], bt.to(dev), lens_t.to(dev), 128 ** -0.5,
        *[d.to(dev) if d is not None else None for d in ds], out=out, return_softmax_lse=True,
        num_splits=num_splits, q_len=q_len, cu_seqlens_q=torch.from_numpy(cu).to(dev) if ragged else None,
        causal=causal)
    npd = [None if d is None else d.numpy() for d in ds]
    exp, lse_exp = O.paged_decode_attention(raw(q), q_dtype, raw(fused[:, 0]), raw(fused[:, 1]), bt.numpy(),
                                            lens_t.numpy(), 128 ** -0.5, *npd, cu_seqlens_q=cu, causal=causal)
    vd_max = 1.0 if npd[2] is None else float(np.max(npd[2]))
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max()) * vd_max
    _check(got, exp, vmax, out_dtype == torch.bfloat16)
    lse_got = lse.cpu().numpy().T.astype(np.float64)
    fin = np.isfinite(lse_exp)
    assert np.isneginf(lse_got[~fin]).all()
    lse_err = np.abs(lse_got[fin] - lse_exp[fin])
    assert (lse_err <= 5e-4 + 1e-5 * np.abs(lse_exp[fin])).all(), f"lse max err {lse_err.max():.3e}"
    return got


LENS = [0, 1, 2, 3, 15, 16, 17, 100, 513, 1500]


@pytest.mark.parametrize(
    "Hq,Hkv,ps,q_len,causal,q_dtype,out_dtype",
    [
        (8, 2, 16, 4, True, "bf16", torch.float32),      # 16 rows: 4 tokens x 4 heads
        (32, 8, 16, 2, True, "fp8", torch.bfloat16),     # 8 rows
        (16, 2, 64, 2, True, "bf16", torch.float32),     # 16 rows: 2 tokens x 8 heads
        (4, 4, 24, 3, True, "bf16", torch.float32),      # general pages, 3 rows
        (12, 6, 16, 5, False, "bf16", torch.float32),    # 10 rows, no mask
        (8, 8, 16, 16, True, "fp8", torch.float32),      # 16 tokens of one head
        (6, 2, 32, 5, True, "bf16", torch.bfloat16),     # 15 rows
        (4, 1, 5, 4, True, "bf16", torch.float32),       # pages of 5, 16 rows
    ],
)
def test_spec_decode_matches_oracle(dev, Hq, Hkv, ps, q_len, causal, q_dtype, out_dtype):
    rng = np.random.default_rng(Hq * 100 + q_len)
    counts = rng.integers(1, q_len + 1, len(LENS)).tolist()
    counts[-1] = q_len
    _spec_case(dev, 7 + Hq + ps + q_len, LENS, counts, Hq, Hkv, ps, q_len, causal, q_dtype, out_dtype)


@pytest.mark.parametrize("q_len", [2, 4])
@pytest.mark.parametrize("num_splits", [0, 1, 3, 40])
def test_spec_decode_schedules(dev, q_len, num_splits):
    """Uniform q_len (no cu_seqlens_q) over the balanced schedule and explicit
    split counts: the causal band falls inside whichever workgroup holds a
    sequence's last tile."""
    _spec_case(dev, 50 + num_splits, LENS, None, 8, 2, 16, q_len, True, num_splits=num_splits, ragged=False)


@pytest.mark.parametrize("ps", [16, 12])
def test_spec_decode_single_long_sequence(dev, ps):
    """One sequence (the per-head balanced kernel) spread over every run."""
    _spec_case(dev, 71 + ps, [20000], [4], 8, 2, ps, 4, True)


def test_spec_decode_last_token_equals_plain_decode(dev):
    """The last query token of each sequence sees every key: its output equals
    a one-token decode of the same query rows up to the order of the fp32
    merges (the two calls split the tiles into different runs)."""
    lens = [40, 700, 1, 3000, 16]
    q_len = 3
    got = _spec_case(dev, 91, lens, [q_len] * len(lens), 8, 2, 16, q_len, True, ragged=False, descales=False)
    g = torch.Generator().manual_seed(91)
    # rebuild the same inputs as _spec_case made them
    P = max(64, sum(-(-x // 16) for x in lens) + 8)
    fused = torch.zeros(P, 2, 16, 2, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, 16, 2, 128), 2.0, g)
    fused[:, 1] = _fp8((P, 16, 2, 128), 2.0, g)
    W = max(-(-x // 16) for x in lens)
    bt = torch.stack([torch.randperm(P, generator=g)[:W] for _ in range(len(lens))]).to(torch.int32)
    q = (torch.randn(q_len * len(lens), 8, 128, generator=g) * 3).to(torch.bfloat16)
    fd = fused.to(dev)
    last = q.view(len(lens), q_len, 8, 128)[:, -1].contiguous().to(dev)
    one = attention.paged_decode_attention(last, fd[:, 0], fd[:, 1], bt.to(dev),
                                           torch.tensor(lens, dtype=torch.int32, device=dev), 128 ** -0.5,
                                           out=torch.empty(len(lens), 8, 128, device=dev))
    spec_last = got.view(len(lens), q_len, 8, 128)[:, -1]
    err = (spec_last - one).abs().max().item()
    assert err <= 1e-5 * max(1.0, one.abs().max().item()), err


def test_flash_attn_varlen_func_spec_decode(dev):
    """The FA3 entry with max_seqlen_q > 1 and ragged cu_seqlens_q, as the
    reference's _fp8_paged_attn calls it for a batch of draft tokens."""
    g = torch.Generator().manual_seed(8)
    P, ps, H, Hq = 300, 16, 4, 16
    fused = torch.zeros(P, 2, ps, H, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, H, 128), 1.0, g)
    fused[:, 1] = _fp8((P, ps, H, 128), 1.0, g)
    fd = fused.to(dev)
    B = 3
    bt = torch.stack([torch.randperm(P, generator=g)[:40] for _ in range(B)]).to(torch.int32).to(dev)
    lens = torch.tensor([5, 300, 640], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 2, 3, 7], dtype=torch.int32, device=dev)
    q = (torch.randn(7, Hq, 128, generator=g)).to(torch.bfloat16).clamp(-448, 448).to(torch.float8_e4m3fn).to(dev)
    one = torch.ones((), dtype=torch.float32, device=dev)
    descale = one.expand(B, H)
    a = attention.flash_attn_varlen_func(
        q=q, k=fd[:, 0], v=fd[:, 1], max_seqlen_q=4, cu_seqlens_q=cu, max_seqlen_k=None, seqused_k=lens,
        block_table=bt, softmax_scale=0.1, causal=True, fa_version=3, q_descale=descale, k_descale=descale,
        v_descale=descale)
    b = attention.paged_decode_attention(q, fd[:, 0], fd[:, 1], bt, lens, 0.1, q_len=4, cu_seqlens_q=cu, causal=True)
    assert torch.equal(a, b)
    exp, _ = O.paged_decode_attention(raw(q), "fp8", raw(fused[:, 0]), raw(fused[:, 1]), bt.cpu().numpy(),
                                      lens.cpu().numpy(), 0.1, cu_seqlens_q=cu.cpu().numpy(), causal=True)
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max())
    _check(a, exp, vmax, True)


def test_flash_attn_varlen_func_sequences_without_query_tokens(dev):
    """max_seqlen_q == 1 with sequences that have no query token this step
    (cu_seqlens_q repeats a value): their rows do not exist in q, and the
    other sequences' rows are read and written where cu_seqlens_q puts them."""
    g = torch.Generator().manual_seed(9)
    P, ps, H, Hq = 200, 16, 2, 8
    fused = torch.zeros(P, 2, ps, H, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, H, 128), 1.0, g)
    fused[:, 1] = _fp8((P, ps, H, 128), 1.0, g)
    fd = fused.to(dev)
    B = 5
    bt = torch.stack([torch.randperm(P, generator=g)[:30] for _ in range(B)]).to(torch.int32).to(dev)
    lens = torch.tensor([40, 300, 7, 480, 33], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 1, 1, 2, 2, 3], dtype=torch.int32, device=dev)
    q = (torch.randn(3, Hq, 128, generator=g)).to(torch.bfloat16).to(dev)
    print("varlen decode with empty query rows", flush=True)
    a = attention.flash_attn_varlen_func(q=q, k=fd[:, 0], v=fd[:, 1], max_seqlen_q=1, cu_seqlens_q=cu,
                                         seqused_k=lens, block_table=bt, softmax_scale=0.1, causal=True)
    assert a.shape == (3, Hq, 128)
    exp, _ = O.paged_decode_attention(raw(q), "bf16", raw(fused[:, 0]), raw(fused[:, 1]), bt.cpu().numpy(),
                                      lens.cpu().numpy(), 0.1, cu_seqlens_q=cu.cpu().numpy(), causal=True)
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max())
    _check(a, exp, vmax, True)


@pytest.mark.parametrize("seed", range(10))
def test_spec_decode_random_shapes(dev, seed):
    """Seeded random batches: 1-16 query tokens per sequence times 1-8 heads
    per kv head within 16 rows, ragged or uniform, causal or not, power-of-two
    and other page sizes, 1-40 sequences of 0-3000 tokens, the balanced and
    split schedules, fp8 and bf16 queries and outputs."""
    rng = np.random.default_rng(3000 + seed)
    G = int(rng.choice([1, 2, 3, 4, 5, 8]))
    q_len = int(rng.integers(1, 16 // G + 1))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    ps = int(rng.choice([16, 32, 64, 24, 5]))
    B = int(rng.choice([1, 2, 3, 7, 13, 40]))
    lens = rng.integers(0, 3000, B).tolist()
    lens[int(rng.integers(0, B))] = int(rng.integers(1, 3000))
    ragged = bool(seed % 2)
    counts = rng.integers(0 if ragged else 1, q_len + 1, B).tolist()
    causal = seed % 3 != 2
    num_splits = 0 if seed % 4 else int(rng.integers(1, 24))
    q_dtype = "fp8" if seed % 5 < 2 else "bf16"
    out_dtype = torch.float32 if seed % 2 else torch.bfloat16
    print(f"spec random {seed}: G={G} q_len={q_len} Hkv={Hkv} ps={ps} B={B} ragged={ragged} causal={causal} "
          f"splits={num_splits}", flush=True)
    _spec_case(dev, 4000 + seed, lens, counts, G * Hkv, Hkv, ps, q_len, causal, q_dtype, out_dtype,
               num_splits=num_splits, ragged=ragged)


def test_reference_fp8_paged_attn_call_through_fp8_kv(dev):
    """The reference's _fp8_paged_attn (pipeswift/llms/layers/attention.py:
    148-187) restated call for call on this package's fp8_kv: quantize the
    query, unit descales as a stride-0 view, attn_varlen_func() with the FA3
    keywords, decode and 2-token steps in one ragged batch."""
    from pipeswift_amd import fp8_kv

    g = torch.Generator().manual_seed(12)
    P, ps, H, Hq = 300, 16, 4, 16
    fused = torch.zeros(P, 2, ps, H, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, H, 128), 1.0, g)
    fused[:, 1] = _fp8((P, ps, H, 128), 1.0, g)
    fd = fused.to(dev)
    B = 4
    bt = torch.stack([torch.randperm(P, generator=g)[:40] for _ in range(B)]).to(torch.int32).to(dev)
    lens = torch.tensor([17, 300, 640, 2], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 1, 3, 5, 6], dtype=torch.int32, device=dev)
    query = (torch.randn(6, Hq, 128, generator=g) * 2).to(torch.bfloat16).to(dev)
    fp8_kv.check_available()
    fp8_kv.warmup(dev)
    descale = fp8_kv.unit_descale(cu.shape[0] - 1, fd.shape[3], dev)
    assert descale.shape == (B, H) and descale.stride() == (0, 0)
    print("reference-style fp8 paged attention call", flush=True)
    out = fp8_kv.attn_varlen_func()(
        q=fp8_kv.quantize(query), k=fd[:, 0], v=fd[:, 1], max_seqlen_q=2, cu_seqlens_q=cu, max_seqlen_k=None,
        seqused_k=lens, block_table=bt, softmax_scale=0.0883883, causal=True, fa_version=3,
        q_descale=descale, k_descale=descale, v_descale=descale, return_softmax_lse=False)
    q8 = fp8_kv.quantize(query)
    exp, _ = O.paged_decode_attention(raw(q8), "fp8", raw(fused[:, 0]), raw(fused[:, 1]), bt.cpu().numpy(),
                                      lens.cpu().numpy(), 0.0883883, cu_seqlens_q=cu.cpu().numpy(), causal=True)
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max())
    _check(out, exp, vmax, True)
