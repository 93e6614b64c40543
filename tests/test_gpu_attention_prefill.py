"""GPU parity of prefill over the paged FP8 cache: ``flash_attn_varlen_func``
with more query rows per kv head than one MFMA tile of the decode reader
holds (``max_seqlen_q * Hq / Hkv > 16``), which the reference's
``_fp8_paged_attn`` passes for every prefill step (attention.py:577-585).
Those steps run ``psk_paged_prefill_attention``; its arithmetic per row is
the decode reader's (exact FP8 -> bf16 Q K^T operands, fp32 MFMA sums) except
that P V takes P rounded once to fp16 (V exactly as fp16) where the decode
reader keeps ~16 bits of P in a bf16 hi + lo pair.  The tolerances are the
decode reader's (see test_gpu_attention.py) plus what the fp16 rounding of
P can add:
  * output: |got - oracle| <= 3e-4 * vmax + 1e-4 * |oracle|, vmax = max|V * vd|
    (bf16 output: plus the bf16 rounding of the oracle, 2^-8 |oracle|)
    + for the prefill kernel (2^-11 + K * 2^-25) * vmax, K the most keys a
    row sees: each weight p <= 2^15 (relative to the maximum of its row's
    first 32 keys, whose key has p = 1, so the row's sum l >= 1) rounds with
    relative error <= 2^-11 from 2^-14 up and absolute error <= 2^-25 below,
    so sum_i |dp_i| |v_i| / l <= 2^-11 vmax + K 2^-25 vmax
  * lse:    |got - oracle| <= 5e-4 + 1e-5 * |oracle| (the sum l is taken
    over the unrounded p)
The oracle (oracle/kv_oracle.py: paged_decode_attention) runs in float64 over
the same ragged layout and is pinned against torch SDPA under torch's
lower-right causal mask.  The decode reader run over chunks of the same step
(``attention.chunked_prefill_attention``) is a second, independent GPU path
that must agree with both.
"""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd import attention, fp8_kv
from tests.conftest import raw

pytestmark = pytest.mark.gpu


_Q_NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32", torch.float8_e4m3fn: "fp8"}


def _prefill_case(dev, seed, lens, counts, Hq, Hkv, ps, causal, descales=True, num_splits=0, spare_rows=0,
                  out_dtype=torch.float32, q_dtype=torch.bfloat16, path="entry", scale=128 ** -0.5, k_sign=1.0,
                  bad_ids=False):
    """One ragged step through ``path`` ("entry": flash_attn_varlen_func as
    the reference calls it; "prefill": paged_prefill_attention directly;
    "chunks": the decode reader over chunks), checked against the oracle."""
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    P = max(64, sum(-(-x // ps) for x in lens) + 8)
    fused = torch.zeros(P, 2, ps, Hkv, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = (torch.randn((P, ps, Hkv, 128), generator=g) * 2.0).to(torch.float8_e4m3fn)
    fused[:, 1] = (torch.randn((P, ps, Hkv, 128), generator=g) * 2.0).to(torch.float8_e4m3fn)
    W = max(1, max(-(-x // ps) for x in lens))
    bt = torch.stack([torch.randperm(P, generator=g)[:W] for _ in range(B)]).to(torch.int32)
    if bad_ids:  # missing pages inside the sequences: their rows read as zeros
        for b in range(B):
            used = -(-lens[b] // ps)
            if used > 1:
                bt[b, 1] = -3 if b % 2 else P + 5
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    TQ = int(cu[-1]) + spare_rows
    q = (torch.randn(TQ, Hq, 128, generator=g) * 3)
    q = q.clamp(-448, 448).to(q_dtype)
    rng = np.random.default_rng(seed)
    ds = [torch.from_numpy(rng.uniform(0.5, 2.0, (B, Hkv)).astype(np.float32)) for _ in range(3)] if descales \
        else [None] * 3
    if k_sign != 1.0:
        ds[1] = ds[1] * k_sign
    fd = fused.to(dev)
    out = torch.full((TQ, Hq, 128), 7.0, dtype=out_dtype, device=dev)
    print(f"prefill case seed={seed} B={B} counts={list(counts)[:8]} Hq={Hq} Hkv={Hkv} ps={ps} causal={causal} "
          f"splits={num_splits} out={out_dtype} q={q_dtype} path={path}", flush=True)
    dd = [None if d is None else d.to(dev) for d in ds]
    kw = dict(softmax_scale=scale, causal=causal, q_descale=dd[0], k_descale=dd[1], v_descale=dd[2],
              return_softmax_lse=True, out=out)
    cu_d = torch.from_numpy(cu).to(dev)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
    if path == "entry":
        f = fp8_kv.attn_varlen_func()
        got, lse = f(q=q.to(dev), k=fd[:, 0], v=fd[:, 1], max_seqlen_q=int(max(counts)), cu_seqlens_q=cu_d,
                     max_seqlen_k=None, seqused_k=lens_d, block_table=bt.to(dev), num_splits=num_splits, **kw)
    elif path == "prefill":
        got, lse = attention.paged_prefill_attention(q.to(dev), fd[:, 0], fd[:, 1], bt.to(dev), lens_d, cu_d,
                                                     int(max(counts)), **kw)
    else:
        got, lse = attention.chunked_prefill_attention(q.to(dev), fd[:, 0], fd[:, 1], int(max(counts)), cu_d, lens_d,
                                                       bt.to(dev), num_splits=num_splits, **kw)
    npd = [None if d is None else d.numpy() for d in ds]
    exp, lse_exp = O.paged_decode_attention(raw(q[: int(cu[-1])]), _Q_NAMES[q_dtype], raw(fused[:, 0]),
                                            raw(fused[:, 1]), bt.numpy(), np.array(lens), scale, *npd,
                                            cu_seqlens_q=cu, causal=causal)
    n = int(cu[-1])
    vd_max = 1.0 if npd[2] is None else float(np.max(npd[2]))
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max()) * vd_max
    gotn = got[:n].double().cpu().numpy()
    err = np.abs(gotn - exp)
    tol = 3e-4 * vmax + 1e-4 * np.abs(exp)
    if _runs_prefill_kernel(path, counts, Hq, Hkv):
        tol = tol + p_rounding_bound(max(lens), vmax)
    if out_dtype == torch.bfloat16:
        tol = tol + 2.0 ** -8 * np.abs(exp)
    assert (err <= tol).all(), f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"
    lse_got = lse.cpu().numpy().T.astype(np.float64)[:n]
    fin = np.isfinite(lse_exp)
    assert np.isneginf(lse_got[~fin]).all()
    lse_err = np.abs(lse_got[fin] - lse_exp[fin])
    assert (lse_err <= 5e-4 + 1e-5 * np.abs(lse_exp[fin])).all(), f"lse max err {lse_err.max():.3e}"
    if spare_rows:  # rows past the last sequence are not written
        assert bool((got[n:] == 7.0).all())
    return got, vmax


def _runs_prefill_kernel(path, counts, Hq, Hkv):
    """Whether the step runs the prefill kernel (flash_attn_varlen_func's
    routing: more than 16 query rows per kv head)."""
    return path == "prefill" or (path == "entry" and max(counts) * max(Hq // Hkv, 1) > 16)


def p_rounding_bound(keys, vmax):
    """What rounding P to fp16 can add to an output of the prefill kernel
    (the module docstring derives it)."""
    return (2.0 ** -11 + keys * 2.0 ** -25) * vmax


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 8), (8, 8), (16, 1), (32, 1), (6, 2), (256, 2)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ragged(dev, Hq, Hkv, causal):
    """Prefill and chunked prefill: sequences with 1 to 200 query tokens over
    prefixes of 0 to 900 cached tokens (the query tokens are each sequence's
    last positions), groups of 1 to 128 query heads per kv head (3: rows of a
    token straddle MFMA row sets; 128: two query tokens per block), so one to
    a hundred query blocks per sequence."""
    rng = np.random.default_rng(Hq * 10 + Hkv + causal)
    B = 7
    counts = [int(x) for x in rng.integers(1, 200, B)]
    counts[2] = 1  # a decode-sized sequence in the same batch
    lens = [c + int(p) for c, p in zip(counts, rng.integers(0, 900, B))]
    lens[4] = counts[4]  # no prefix: the whole sequence is new
    _prefill_case(dev, 500 + Hq + Hkv + causal, lens, counts, Hq, Hkv, 16, causal)


@pytest.mark.parametrize("ps", [16, 24, 64])
def test_prefill_block_sizes(dev, ps):
    """Other page sizes (24: page rows found by division), empty sequences
    and spare query rows past the last one; the decode reader over chunks of
    the same step (with an explicit split count) agrees as well."""
    counts = [40, 0, 130, 17, 0, 64]
    lens = [40 + 300, 12, 130, 17 + 5, 0, 64 + 1000]
    a, vmax = _prefill_case(dev, 600 + ps, lens, counts, 32, 8, ps, True, spare_rows=5)
    b, _ = _prefill_case(dev, 600 + ps, lens, counts, 32, 8, ps, True, spare_rows=5, path="chunks", num_splits=3)
    n = sum(counts)
    # each within its tolerance of the oracle, so within their sum of each other
    bound = 2 * (3e-4 * vmax + 1e-4 * float(b[:n].abs().max())) + p_rounding_bound(max(lens), vmax)
    assert float((a[:n] - b[:n]).abs().max()) <= bound


def test_prefill_group_16_over_1100_tokens(dev):
    """A chunked-prefill step of 1100 new tokens over 6 sequences with prefixes
    up to 1500 tokens at 16 query heads over one kv head (16-token query
    blocks); unit descales, as the reference passes them.  Through the decode
    reader the same step is 1100+ one-token chunk sequences, past its balanced
    schedule's 1024, which its split schedule reads."""
    rng = np.random.default_rng(77)
    cuts = np.sort(rng.choice(np.arange(1, 1100), 5, replace=False))
    counts = np.diff(np.concatenate([[0], cuts, [1100]])).tolist()
    lens = [int(c) + int(p) * 16 for c, p in zip(counts, rng.integers(0, 94, 6))]
    _prefill_case(dev, 700, lens, counts, 16, 1, 16, True, descales=False)
    _prefill_case(dev, 700, lens, counts, 16, 1, 16, True, descales=False, path="chunks")


def test_prefill_shorter_sequence_than_its_queries(dev):
    """Query tokens past the sequence's keys see no key: zeros and lse -inf, as
    in the decode reader (FA's bottom-right alignment)."""
    _prefill_case(dev, 800, [5, 300], [20, 40], 32, 8, 16, True)


@pytest.mark.parametrize("q_dtype,out_dtype", [(torch.float8_e4m3fn, torch.float32), (torch.float16, torch.float32),
                                               (torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16)])
def test_prefill_query_and_output_dtypes(dev, q_dtype, out_dtype):
    """An FP8 query is used as is, the others quantized as e4m3(q / qd);
    bf16 or float32 output; through paged_prefill_attention directly."""
    _prefill_case(dev, 900, [300, 77, 500], [120, 77, 33], 32, 4, 16, True, q_dtype=q_dtype, out_dtype=out_dtype,
                  path="prefill")


def test_prefill_many_sequences(dev):
    """150 sequences of 1 to 40 query tokens (the block search's two rounds),
    at 8 query heads per kv head."""
    rng = np.random.default_rng(91)
    counts = [int(x) for x in rng.integers(1, 40, 150)]
    lens = [c + int(p) for c, p in zip(counts, rng.integers(0, 200, 150))]
    _prefill_case(dev, 901, lens, counts, 16, 2, 16, True)


def test_prefill_long_prefix(dev):
    """Config 3's shape at a smaller scale: 600 and 900 new tokens over
    prefixes of 2000 and 4000 cached tokens, 32 query heads over 4 kv heads,
    many stages per workgroup and the causal band across two of them."""
    _prefill_case(dev, 902, [2600, 4900], [600, 900], 32, 4, 16, True)


def test_prefill_steep_scores_take_the_exact_redo(dev):
    """Scores spread over hundreds of binary orders of magnitude (softmax
    scale 4): rows pass the prefill kernel's 2^15 headroom above the maximum
    of their first 32 keys, so their workgroups recompute with exact row
    maxima; results still match the float64 oracle."""
    _prefill_case(dev, 903, [700, 90, 1500], [300, 90, 64], 32, 4, 16, True, scale=4.0)


def test_prefill_negative_score_scale(dev):
    """A negative k descale (the score scale's sign applied to q~, exactly)."""
    _prefill_case(dev, 904, [400, 250], [120, 250], 16, 2, 16, True, k_sign=-1.0)


def test_prefill_missing_pages_read_as_zero_rows(dev):
    """Block-table entries outside [0, num_blocks) inside the sequences read
    as zero K and V rows (scores 0), as in the decode reader and the oracle."""
    _prefill_case(dev, 905, [300, 200, 90], [100, 200, 40], 32, 8, 16, True, bad_ids=True)


def test_prefill_page_stride_past_32_bits(dev):
    """Pages 4 GiB + 32 KiB apart (a strided view over one allocation): the
    loader's 64-bit offset path, which strides below 2^32 never take."""
    Hkv, Hq, ps, D = 2, 16, 16, 128
    stride = (1 << 32) + (1 << 15)
    base = torch.zeros(stride + 2 * ps * Hkv * D * 2, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(906)
    pages = (torch.randn(2, 2, ps, Hkv, D, generator=g) * 2).to(torch.float8_e4m3fn)  # [page, K/V, row, head, d]
    for p in range(2):
        base[p * stride: p * stride + 2 * ps * Hkv * D].copy_(pages[p].reshape(-1).view(torch.uint8).to(dev))
    kc = base.view(torch.float8_e4m3fn).as_strided((2, ps, Hkv, D), (stride, Hkv * D, D, 1))
    vc = base.view(torch.float8_e4m3fn).as_strided((2, ps, Hkv, D), (stride, Hkv * D, D, 1), ps * Hkv * D)
    L, n = 30, 20
    q = (torch.randn(n, Hq, D, generator=g) * 3).to(torch.bfloat16)
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    cu = torch.tensor([0, n], dtype=torch.int32)
    print(f"prefill wide page stride: stride={stride}", flush=True)
    got = attention.paged_prefill_attention(q.to(dev), kc, vc, bt.to(dev), torch.tensor([L], dtype=torch.int32,
                                            device=dev), cu.to(dev), n, 128 ** -0.5,
                                            out=torch.zeros(n, Hq, D, dtype=torch.float32, device=dev))
    exp, _ = O.paged_decode_attention(raw(q), "bf16", raw(pages[:, 0]), raw(pages[:, 1]), bt.numpy(), np.array([L]),
                                      128 ** -0.5, cu_seqlens_q=cu.numpy(), causal=True)
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(pages[:, 1]))).max())
    err = np.abs(got.double().cpu().numpy() - exp)
    assert (err <= 3e-4 * vmax + p_rounding_bound(L, vmax) + 1e-4 * np.abs(exp)).all(), f"max err {err.max():.3e}"


def test_prefill_weights_at_the_edge_of_fp16(dev):
    """A key 2^14.9, 2^15.8 and 2^17 times heavier than the first 32 keys of
    its row (one sequence each): the first weight is a large but finite fp16
    value on the pass without rescale; the second is finite in fp16 but past
    the 2^15 headroom, and the third overflows fp16, so those workgroups
    must take the exact redo.  Scores are q~0 * K0 * kd in the exp2 domain
    (softmax scale ln 2, every other q and K element 0): K0 = 16 at key 40
    of 64 and 0 elsewhere, q~0 the E4M3 query from -1 to 1 over a sequence's
    rows, kd = 14.9/16, 15.8/16, 17/16 by sequence.  Results match the
    float64 oracle, finite everywhere."""
    ps, D, L, n = 16, 128, 64, 20
    g = torch.Generator().manual_seed(908)
    P = 3 * L // ps + 2
    kf = torch.zeros(P, ps, 1, D)
    for b in range(3):
        kf[b * 4 + 2, 40 - 32, 0, 0] = 16.0  # key 40 of sequence b (page 2 of its 4)
    kc8 = kf.to(torch.float8_e4m3fn)
    vc8 = (torch.randn(P, ps, 1, D, generator=g) * 2).to(torch.float8_e4m3fn)
    q = torch.zeros(3 * n, 1, D)
    q[:, 0, 0] = torch.linspace(-1.0, 1.0, n).repeat(3)
    q = q.to(torch.bfloat16)
    kd = torch.tensor([[14.9 / 16], [15.8 / 16], [17.0 / 16]], dtype=torch.float32)
    bt = torch.arange(12, dtype=torch.int32).view(3, 4)
    cu = torch.tensor([0, n, 2 * n, 3 * n], dtype=torch.int32)
    lens = torch.full((3,), L, dtype=torch.int32)
    scale = float(np.log(2.0))
    print("prefill fp16 weight edge: 3 sequences, key 40 at 14.9/15.8/17 binades", flush=True)
    got = attention.paged_prefill_attention(q.to(dev), kc8.to(dev), vc8.to(dev), bt.to(dev), lens.to(dev), cu.to(dev),
                                            n, scale, None, kd.to(dev), None,
                                            out=torch.zeros(3 * n, 1, D, dtype=torch.float32, device=dev),
                                            causal=False)
    exp, _ = O.paged_decode_attention(raw(q), "bf16", raw(kc8), raw(vc8), bt.numpy(), lens.numpy(), scale, None,
                                      kd.numpy(), None, cu_seqlens_q=cu.numpy(), causal=False)
    gotn = got.double().cpu().numpy()
    assert np.isfinite(gotn).all()
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(vc8))).max())
    err = np.abs(gotn - exp)
    assert (err <= 3e-4 * vmax + p_rounding_bound(L, vmax) + 1e-4 * np.abs(exp)).all(), f"max err {err.max():.3e}"


def test_prefill_more_sequences_than_the_pre_pass_orders(dev):
    """1100 sequences of 2 to 4 query tokens (past the pre-pass's 1024, which
    then keeps batch order; the block search takes two rounds), a few of them
    without query tokens."""
    rng = np.random.default_rng(907)
    counts = [int(x) for x in rng.integers(2, 5, 1100)]
    for b in (5, 600, 1099):
        counts[b] = 0
    lens = [c + int(p) for c, p in zip(counts, rng.integers(0, 60, 1100))]
    _prefill_case(dev, 907, lens, counts, 32, 4, 16, True)


def test_prefill_bench_step_matches_decode_reader(dev):
    """The bench's prefill_attention step at full size (config 3 geometry:
    4096 query tokens over 6 sequences with 14k-45k cached keys, 32 query
    heads over 4 kv heads, random FP8 pages, per-tensor descales, the bench's
    seeds): the prefill kernel against the decode reader over 2-token chunks
    of the same step, float32 outputs.  Two independent kernels, each pinned
    to the oracle at smaller sizes, agree to 1e-3 of the largest output."""
    import workloads

    cc = workloads.config3_chunked()
    H, D, Hq, ps = 4, 128, 32, 16
    P = cc.append.cache.shape[0]
    g = torch.Generator(device=dev).manual_seed(76)
    cache = (torch.randn((P, 2, ps, H, D), device=dev, generator=g) * 2.0).to(torch.float8_e4m3fn)
    kc, vc = cache[:, 0], cache[:, 1]
    bt = cc.block_table.to(dev)
    N = int(cc.chunk.sum())
    cu = torch.zeros(len(cc.chunk) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(cc.chunk, 0).to(torch.int32)
    cu = cu.to(dev)
    lens = (cc.prefix + cc.chunk).to(torch.int32).to(dev)
    q = (torch.randn(N, Hq, D, device=dev, generator=g) * 2.0).to(torch.bfloat16)
    kd = torch.tensor([0.01], dtype=torch.float32, device=dev)
    vd = torch.tensor([0.02], dtype=torch.float32, device=dev)
    maxq = int(cc.chunk.max())
    print(f"prefill bench step: N={N} keys={int(lens.sum())} P={P}", flush=True)
    a = torch.empty(N, Hq, D, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    attention.paged_prefill_attention(q, kc, vc, bt, lens, cu, maxq, D ** -0.5, None, kd, vd, out=a, causal=True)
    attention.chunked_prefill_attention(q, kc, vc, maxq, cu, lens, bt, softmax_scale=D ** -0.5, causal=True,
                                        k_descale=kd, v_descale=vd, out=b)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(a).all())
    ref = float(b.abs().max())
    assert ref > 0.0 and float((a - b).abs().max()) <= 1e-3 * ref
