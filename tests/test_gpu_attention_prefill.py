"""GPU parity of prefill over the paged FP8 cache: ``flash_attn_varlen_func``
with more query tokens per sequence than one MFMA tile holds
(``max_seqlen_q * Hq / Hkv > 16``), which the reference's
``_fp8_paged_attn`` passes for every prefill step (attention.py:577-585).
Each sequence's query tokens are read in chunks of 16 / G tokens, each a
sequence of its own, so the arithmetic per row is the decode reader's and
so are the tolerances (see test_gpu_attention.py):
  * fp32 output: |got - oracle| <= 3e-4 * max|V * vd| + 1e-4 * |oracle|
  * lse:         |got - oracle| <= 5e-4 + 1e-5 * |oracle|
The oracle (oracle/kv_oracle.py: paged_decode_attention) runs in float64 over
the same ragged layout and is pinned against torch SDPA under torch's
lower-right causal mask.
"""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd import fp8_kv
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def _prefill_case(dev, seed, lens, counts, Hq, Hkv, ps, causal, descales=True, num_splits=0, spare_rows=0):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    P = max(64, sum(-(-x // ps) for x in lens) + 8)
    fused = torch.zeros(P, 2, ps, Hkv, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = (torch.randn((P, ps, Hkv, 128), generator=g) * 2.0).to(torch.float8_e4m3fn)
    fused[:, 1] = (torch.randn((P, ps, Hkv, 128), generator=g) * 2.0).to(torch.float8_e4m3fn)
    W = max(1, max(-(-x // ps) for x in lens))
    bt = torch.stack([torch.randperm(P, generator=g)[:W] for _ in range(B)]).to(torch.int32)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    TQ = int(cu[-1]) + spare_rows
    q = (torch.randn(TQ, Hq, 128, generator=g) * 3).to(torch.bfloat16)
    rng = np.random.default_rng(seed)
    ds = [torch.from_numpy(rng.uniform(0.5, 2.0, (B, Hkv)).astype(np.float32)) for _ in range(3)] if descales \
        else [None] * 3
    fd = fused.to(dev)
    out = torch.full((TQ, Hq, 128), 7.0, dtype=torch.float32, device=dev)
    print(f"prefill case seed={seed} B={B} counts={list(counts)[:8]} Hq={Hq} Hkv={Hkv} ps={ps} causal={causal} "
          f"splits={num_splits}", flush=True)
    f = fp8_kv.attn_varlen_func()
    got, lse = f(q=q.to(dev), k=fd[:, 0], v=fd[:, 1], max_seqlen_q=int(max(counts)),
                 cu_seqlens_q=torch.from_numpy(cu).to(dev), max_seqlen_k=None,
                 seqused_k=torch.tensor(lens, dtype=torch.int32, device=dev), block_table=bt.to(dev),
                 softmax_scale=128 ** -0.5, causal=causal, q_descale=None if ds[0] is None else ds[0].to(dev),
                 k_descale=None if ds[1] is None else ds[1].to(dev), v_descale=None if ds[2] is None else ds[2].to(dev),
                 return_softmax_lse=True, out=out, num_splits=num_splits)
    npd = [None if d is None else d.numpy() for d in ds]
    exp, lse_exp = O.paged_decode_attention(raw(q[: int(cu[-1])]), "bf16", raw(fused[:, 0]), raw(fused[:, 1]),
                                            bt.numpy(), np.array(lens), 128 ** -0.5, *npd, cu_seqlens_q=cu,
                                            causal=causal)
    n = int(cu[-1])
    vd_max = 1.0 if npd[2] is None else float(np.max(npd[2]))
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max()) * vd_max
    gotn = got[:n].double().cpu().numpy()
    err = np.abs(gotn - exp)
    tol = 3e-4 * vmax + 1e-4 * np.abs(exp)
    assert (err <= tol).all(), f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"
    lse_got = lse.cpu().numpy().T.astype(np.float64)[:n]
    fin = np.isfinite(lse_exp)
    assert np.isneginf(lse_got[~fin]).all()
    lse_err = np.abs(lse_got[fin] - lse_exp[fin])
    assert (lse_err <= 5e-4 + 1e-5 * np.abs(lse_exp[fin])).all(), f"lse max err {lse_err.max():.3e}"
    if spare_rows:  # rows past the last sequence are not written
        assert bool((got[n:] == 7.0).all())
    return got


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 8), (8, 8), (16, 1)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ragged_chunks(dev, Hq, Hkv, causal):
    """Prefill and chunked prefill: sequences with 1 to 200 query tokens over
    prefixes of 0 to 900 cached tokens (the query tokens are each sequence's
    last positions), every group size's chunk length (16 / G tokens)."""
    rng = np.random.default_rng(Hq * 10 + Hkv + causal)
    B = 7
    counts = [int(x) for x in rng.integers(1, 200, B)]
    counts[2] = 1  # a decode-sized sequence in the same batch
    lens = [c + int(p) for c, p in zip(counts, rng.integers(0, 900, B))]
    lens[4] = counts[4]  # no prefix: the whole sequence is new
    _prefill_case(dev, 500 + Hq + Hkv + causal, lens, counts, Hq, Hkv, 16, causal)


@pytest.mark.parametrize("ps", [16, 24, 64])
def test_prefill_block_sizes_and_splits(dev, ps):
    """Other page sizes (24: the general-page reader) and an explicit split
    count, with empty sequences and spare query rows past the last one."""
    counts = [40, 0, 130, 17, 0, 64]
    lens = [40 + 300, 12, 130, 17 + 5, 0, 64 + 1000]
    _prefill_case(dev, 600 + ps, lens, counts, 32, 8, ps, True, spare_rows=5)
    _prefill_case(dev, 650 + ps, lens, counts, 32, 8, ps, True, num_splits=3)


def test_prefill_more_chunks_than_the_balanced_schedule_takes(dev):
    """A chunked-prefill step of 1100 new tokens over 6 sequences with prefixes
    up to 1500 tokens at 16 query heads over one kv head: chunks of one token,
    so 1100+ chunk sequences, past the balanced schedule's 1024, and the split
    schedule reads them; unit descales, as the reference passes them."""
    rng = np.random.default_rng(77)
    cuts = np.sort(rng.choice(np.arange(1, 1100), 5, replace=False))
    counts = np.diff(np.concatenate([[0], cuts, [1100]])).tolist()
    lens = [int(c) + int(p) * 16 for c, p in zip(counts, rng.integers(0, 94, 6))]
    _prefill_case(dev, 700, lens, counts, 16, 1, 16, True, descales=False)


def test_prefill_shorter_sequence_than_its_queries(dev):
    """Query tokens past the sequence's keys see no key: zeros and lse -inf, as
    in the decode reader (FA's bottom-right alignment)."""
    _prefill_case(dev, 800, [5, 300], [20, 40], 32, 8, 16, True)
