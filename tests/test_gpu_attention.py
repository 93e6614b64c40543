"""GPU parity of the paged decode-attention reader (psk_paged_decode_attention)
over the FP8 cache.

Tolerances (floating point).  The products q~ k are exact (bf16 MFMA over
exactly converted FP8 values), and each 128-term score is summed in fp32.
P V (power-of-two pages) multiplies V, exact in bf16, by p split into bf16
hi + lo, which carries p to a relative 2^-17 -- far inside the bounds below,
as are the fp32 sums of either P V path:
|ds| <~ 128 * 2^-24 * sum|q~ k| * scale * qd * kd, about 1e-4 at these
magnitudes (FP8 values of std 2-3, descales up to 2).  A
score error shifts its softmax weight by the same relative amount, so:
  * fp32 output: |got - oracle| <= 3e-4 * max|V * vd| + 1e-4 * |oracle|
  * bf16 output: the same plus one bf16 rounding (2^-8 relative)
  * lse:         |got - oracle| <= 5e-4 + 1e-5 * |oracle|
The oracle (oracle/kv_oracle.py: paged_decode_attention) runs in float64; at
config 2's full size a float64 torch restatement on the device stands in for it.
"""

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
import workloads
from pipeswift_amd import attention, cache_ops
from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash
from tests.conftest import raw

pytestmark = pytest.mark.gpu


def _fp8(shape, std, gen):
    return (torch.randn(shape, generator=gen) * std).to(torch.float8_e4m3fn)


def _check(got, exp, vmax, bf16):
    got = got.float().cpu().numpy().astype(np.float64)
    tol = 3e-4 * vmax + (2.0 ** -8 + 1e-4 if bf16 else 1e-4) * np.abs(exp)
    err = np.abs(got - exp)
    assert (err <= tol).all(), f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


def _case(dev, seed, B, Hq, Hkv, ps, P, lens, q_dtype, out_dtype, descales, W=None, bad_ids=False, num_splits=0):
    g = torch.Generator().manual_seed(seed)
    fused = torch.zeros(P, 2, ps, Hkv, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, Hkv, 128), 2.0, g)
    fused[:, 1] = _fp8((P, ps, Hkv, 128), 2.0, g)
    lens = torch.tensor(lens, dtype=torch.int32)
    need = int(-(-int(lens.max()) // ps)) if len(lens) else 1
    W = W or max(need, 1)
    bt = torch.stack([torch.randperm(P, generator=g)[:W] for _ in range(B)]).to(torch.int32)
    if bad_ids:
        bt[0, 0] = -1
        bt[-1, 1] = P + 3
    qb = (torch.randn(B, Hq, 128, generator=g) * 3).to(torch.bfloat16)
    q = qb.clamp(-448, 448).to(torch.float8_e4m3fn) if q_dtype == "fp8" else qb
    rng = np.random.default_rng(seed)
    if descales == "per_seq_head":
        ds = [torch.from_numpy(rng.uniform(0.5, 2.0, (B, Hkv)).astype(np.float32)) for _ in range(3)]
    elif descales == "scalar":
        ds = [torch.tensor([float(rng.uniform(0.5, 2.0))], dtype=torch.float32) for _ in range(3)]
    else:
        ds = [None, None, None]
    fd = fused.to(dev)
    out = torch.empty(B, Hq, 128, dtype=out_dtype, device=dev)
    scale = 128 ** -0.5
    got, lse = attention.paged_decode_attention(
        q.to(dev), fd[:, 0], fd[:, 1], bt.to(dev), lens.to(dev), scale,
        *[d.to(dev) if d is not None else None for d in ds], out=out, return_softmax_lse=True, num_splits=num_splits)
    npd = [None if d is None else np.broadcast_to(d.numpy().reshape(-1, 1) if d.numel() == 1 else d.numpy(),
                                                  (B, Hkv)) for d in ds]
    exp, lse_exp = O.paged_decode_attention(raw(q), q_dtype, raw(fused[:, 0]), raw(fused[:, 1]), bt.numpy(),
                                            lens.numpy(), scale, *npd)
    vd_max = 1.0 if npd[2] is None else float(np.max(npd[2]))
    vmax = float(np.abs(O.e4m3fn_to_f32(raw(fused[:, 1]))).max()) * vd_max
    _check(got, exp, vmax, out_dtype == torch.bfloat16)
    lse_got = lse.cpu().numpy().T.astype(np.float64)
    fin = np.isfinite(lse_exp)
    assert (np.isneginf(lse_got[~fin])).all()
    lse_err = np.abs(lse_got[fin] - lse_exp[fin])
    assert (lse_err <= 5e-4 + 1e-5 * np.abs(lse_exp[fin])).all(), f"lse max err {lse_err.max():.3e}"


LENS = [0, 1, 15, 16, 17, 100, 513, 1500, 2049]


@pytest.mark.parametrize(
    "Hq,Hkv,ps,q_dtype,out_dtype,descales",
    [
        (8, 2, 16, "bf16", torch.float32, "per_seq_head"),
        (4, 4, 16, "fp8", torch.bfloat16, None),
        (4, 2, 8, "bf16", torch.float32, "scalar"),
        (10, 2, 32, "bf16", torch.float32, "per_seq_head"),
        (16, 2, 64, "fp8", torch.float32, "per_seq_head"),
        (6, 2, 24, "bf16", torch.bfloat16, None),
        (32, 8, 16, "fp8", torch.bfloat16, "per_seq_head"),
        (8, 8, 32, "bf16", torch.float32, None),
        (12, 6, 16, "bf16", torch.float32, "scalar"),
    ],
)
def test_decode_attention_matches_oracle(dev, Hq, Hkv, ps, q_dtype, out_dtype, descales):
    _case(dev, 11 + Hq + ps, len(LENS), Hq, Hkv, ps, 700, LENS, q_dtype, out_dtype, descales)


@pytest.mark.parametrize("ps", [16, 24])
@pytest.mark.parametrize("num_splits", [0, 1, 3, 40])
def test_balanced_and_split_schedules(dev, num_splits, ps):
    """num_splits 0 is the balanced schedule (every workgroup an equal run of
    (sequence, kv head, tile) units across sequence boundaries); an explicit
    count splits each sequence, as FA's num_splits.  Pages of 24 tokens take
    the general-page variants of the same kernels."""
    _case(dev, 21, len(LENS), 8, 2, ps, 700, LENS, "bf16", torch.float32, "per_seq_head", num_splits=num_splits)


@pytest.mark.parametrize("ps,G", [(5, 1), (12, 8), (48, 4), (100, 2)])
def test_single_sequence_general_pages(dev, ps, G):
    """One sequence (the per-head balanced kernel) on pages that are not a
    power of two >= 16: tiles straddle pages, each lane addresses its own rows."""
    print(f"single sequence: ps={ps} G={G}", flush=True)
    _case(dev, 41 + ps, 1, 2 * G, 2, ps, 2000, [6001], "fp8", torch.float32, "per_seq_head")


@pytest.mark.parametrize("B,Hkv,long_len", [(300, 1, 40000), (2, 4, 0), (1025, 2, 3000)])
def test_balanced_schedule_skewed_batches(dev, B, Hkv, long_len):
    """Many short sequences (zeros included) around one long one: workgroups
    span many sequences, and the long sequence's records come from hundreds of
    workgroups (the combine takes them 64 at a time).  (2, 4, 0): fewer units
    than workgroups.  1025 sequences: more than the balanced schedule takes, so
    the split schedule runs."""
    rng = np.random.default_rng(B)
    lens = rng.integers(0, 40, B).tolist()
    lens[B // 3] = long_len if long_len else 1
    lens[0] = 0
    P = max(64, sum(-(-x // 16) for x in lens) + 16)
    print(f"skewed: B={B} Hkv={Hkv} long={long_len} pages={P}", flush=True)
    _case(dev, 31 + B, B, 4 * Hkv, Hkv, 16, P, lens, "bf16", torch.float32, None)


@pytest.mark.parametrize("ps", [16, 24, 5])
def test_decode_attention_bad_page_ids_read_as_zero_rows(dev, ps):
    """A -1 and an out-of-range page id: their tokens read as zero K and V rows
    (a whole tile with pages of 16; single tokens of a tile with 24 or 5)."""
    _case(dev, 5, 3, 8, 2, ps, 300, [40, 70, 33], "bf16", torch.float32, None, bad_ids=True)


def test_decode_attention_page_ids_beyond_lds_staging(dev):
    """block_size 1 and a 70000-wide table: a range spans more pages than one
    LDS staging of page ids holds (1024), so it is staged in pieces."""
    _case(dev, 6, 2, 4, 1, 1, 80000, [3000, 1100], "bf16", torch.float32, "per_seq_head", W=70000)


def test_reference_accuracy_gate_constant_values(dev):
    """scripts/check_fp8_kv_backend.py: 131072 tokens, 32 query / 4 kv heads,
    pages of 64, V constant per kv head -> the output is V; the reference
    accepts a drift below 5e-3, this reader is held to 1e-5."""
    kv_len, Hq, Hkv, ps = 131072, 32, 4, 64
    pages = kv_len // ps
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, Hq, 128, device=dev, generator=g).to(torch.bfloat16).to(torch.float8_e4m3fn)
    k = torch.randn(pages, ps, Hkv, 128, device=dev, generator=g).to(torch.bfloat16).to(torch.float8_e4m3fn)
    vals = torch.tensor([1.0, 1.5, 2.0, 3.0], device=dev)
    v = vals.view(1, 1, Hkv, 1).expand(pages, ps, Hkv, 128).contiguous().to(torch.float8_e4m3fn)
    bt = torch.arange(pages, device=dev, dtype=torch.int32)[None]
    out = attention.flash_attn_varlen_func(
        q=q, k=k, v=v, max_seqlen_q=1, cu_seqlens_q=torch.tensor([0, 1], device=dev, dtype=torch.int32),
        max_seqlen_k=None, seqused_k=torch.tensor([kv_len], device=dev, dtype=torch.int32), block_table=bt,
        softmax_scale=128 ** -0.5, causal=True, fa_version=3, num_splits=1,
        q_descale=torch.ones(1, Hkv, device=dev), k_descale=torch.ones(1, Hkv, device=dev),
        v_descale=torch.ones(1, Hkv, device=dev)).float()
    exact = vals.repeat_interleave(Hq // Hkv).view(1, Hq, 1)
    drift = ((out - exact) / exact).abs().max().item()
    assert drift < 1e-5, drift


def _torch_reference(q8, kc, vc, tables, ctx, scale, kd, vd, G):
    """float64 restatement on the device, one sequence at a time."""
    outs = []
    for b in range(len(tables)):
        n = int(ctx[b])
        j = torch.arange(n, device=kc.device)
        pages = tables[b].to(kc.device).long()[j // 16]
        K = kc[pages, j % 16].double()  # [n, H, D]
        V = vc[pages, j % 16].double()
        qq = q8[b].double()  # [Hq, D]
        Kr = K.repeat_interleave(G, dim=1).permute(1, 2, 0).contiguous()  # [Hq, D, n]
        s = torch.matmul(qq[:, None, :], Kr)[:, 0] * (scale * kd)  # [Hq, n]
        p = torch.softmax(s, dim=1)
        Vr = V.repeat_interleave(G, dim=1).permute(1, 0, 2).contiguous()  # [Hq, n, D]
        outs.append(torch.matmul(p[:, None, :], Vr)[:, 0] * vd)
    return torch.stack(outs)


def test_config2_append_then_decode_attention(dev):
    """Config 2 at full size: every context token of the 128 sequences is
    appended to the sentinel-filled [65536, 16, 8, 128] FP8 cache (the slots
    past each sequence's last token keep random bytes, NaN encodings among
    them, which the reader must not let through) with per-tensor scales from
    compute_kv_scales, then one decode step reads it back.  Parity against a
    float64 restatement over the same FP8 cache; the FP8 round trip against
    fp32 attention over the unquantized bf16 K/V is reported and bounded."""
    case = workloads.config2_fp8_decode()
    ctx, tables = case.extra["ctx"], case.extra["tables"]
    B, H, D, Hq = 128, 8, 128, 32
    G = Hq // H
    g = torch.Generator(device=dev).manual_seed(2002)
    total = int(ctx.sum())
    kv = (torch.randn(total, 2, H, D, device=dev, generator=g) * 2.0).to(torch.bfloat16)
    slots = torch.cat([tables[b].long().repeat_interleave(16)[: int(ctx[b])] * 16
                       + torch.arange(int(ctx[b])) % 16 for b in range(B)]).to(dev)
    cache = case.cache.to(dev)
    scales = cache_ops.compute_kv_scales(kv[:, 0], kv[:, 1])
    reshape_and_cache_flash(kv[:, 0], kv[:, 1], cache[:, 0], cache[:, 1], slots, scales[0:1], scales[1:2])
    W = max(len(t) for t in tables)
    bt = torch.zeros(B, W, dtype=torch.int32)
    for b in range(B):
        bt[b, : len(tables[b])] = tables[b].to(torch.int32)
    q = case.qkv[:, : Hq * D].view(B, Hq, D).to(dev)
    lens = ctx.to(torch.int32).to(dev)
    scale = D ** -0.5
    ks, vs = scales[0:1], scales[1:2]
    out = torch.empty(B, Hq, D, dtype=torch.float32, device=dev)
    attention.paged_decode_attention(q, cache[:, 0], cache[:, 1], bt.to(dev), lens, scale, None, ks, vs, out=out)
    q8 = q.clamp(-448, 448).to(torch.float8_e4m3fn)
    ref = _torch_reference(q8, cache[:, 0], cache[:, 1], tables, ctx, scale, float(ks), float(vs), G)
    # the cache is sentinel-filled: slots past each sequence's last token hold
    # random bytes (NaN patterns included), which the reader must mask
    vmax = float(kv[:, 1].float().abs().max())
    err = (out.double() - ref).abs()
    assert bool((err <= 3e-4 * vmax + 1e-4 * ref.abs()).all()), float(err.max())
    # FP8 round trip: against fp32 attention over the bf16 K/V and bf16 query.
    # The reader must add nothing to what FP8 storage itself costs: per
    # sequence, its deviation stays within that of exact attention over the
    # same FP8 cache (the float64 restatement), plus 1e-3.
    off = torch.cumsum(torch.cat([torch.zeros(1, dtype=torch.int64), ctx[:-1]]), 0)
    e_read, e_store = [], []
    for b in range(B):
        n = int(ctx[b])
        K = kv[off[b]: off[b] + n, 0].float().repeat_interleave(G, dim=1).permute(1, 2, 0).contiguous()
        V = kv[off[b]: off[b] + n, 1].float().repeat_interleave(G, dim=1).permute(1, 0, 2).contiguous()
        p = torch.softmax(torch.matmul(q[b].float()[:, None, :], K)[:, 0] * scale, dim=1)
        o = torch.matmul(p[:, None, :], V)[:, 0].double()
        e_read.append(float((out[b].double() - o).norm() / o.norm()))
        e_store.append(float((ref[b] - o).norm() / o.norm()))
    e_read, e_store = np.array(e_read), np.array(e_store)
    print(f"config 2 FP8 storage error vs bf16 attention: median {np.median(e_store):.4f}, "
          f"worst {e_store.max():.4f}; reader minus storage, worst {np.max(e_read - e_store):.2e}")
    assert (e_read <= e_store + 1e-3).all()


def test_decode_attention_replays_in_a_hip_graph(dev):
    g = torch.Generator().manual_seed(3)
    P, ps, H, Hq, B = 400, 16, 2, 8, 5
    fused = torch.zeros(P, 2, ps, H, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, H, 128), 2.0, g)
    fused[:, 1] = _fp8((P, ps, H, 128), 2.0, g)
    fd = fused.to(dev)
    bt = torch.stack([torch.randperm(P, generator=g)[:60] for _ in range(B)]).to(torch.int32).to(dev)
    q = (torch.randn(B, Hq, 128, generator=g) * 3).to(torch.bfloat16).to(dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    ws = torch.empty(attention.workspace_floats(B, Hq, H, 60 * ps), dtype=torch.float32, device=dev)
    out = torch.empty(B, Hq, 128, dtype=torch.float32, device=dev)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        attention.paged_decode_attention(q, fd[:, 0], fd[:, 1], bt, lens, out=out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        attention.paged_decode_attention(q, fd[:, 0], fd[:, 1], bt, lens, out=out, workspace=ws)
    for step in range(4):
        lens.copy_(torch.randint(1, 60 * ps, (B,), generator=g, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        eager = attention.paged_decode_attention(q, fd[:, 0], fd[:, 1], bt, lens,
                                                 out=torch.empty_like(out))
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {step} differs from eager"


def test_flash_attn_varlen_func_matches_direct_call(dev):
    g = torch.Generator().manual_seed(4)
    P, ps, H, Hq, B = 300, 16, 4, 16, 3
    fused = torch.zeros(P, 2, ps, H, 128, dtype=torch.float8_e4m3fn)
    fused[:, 0] = _fp8((P, ps, H, 128), 1.0, g)
    fused[:, 1] = _fp8((P, ps, H, 128), 1.0, g)
    fd = fused.to(dev)
    bt = torch.stack([torch.randperm(P, generator=g)[:40] for _ in range(B)]).to(torch.int32).to(dev)
    lens = torch.tensor([5, 300, 640], dtype=torch.int32, device=dev)
    q = (torch.randn(B, Hq, 128, generator=g)).to(torch.bfloat16).clamp(-448, 448).to(torch.float8_e4m3fn).to(dev)
    one = torch.ones((), dtype=torch.float32, device=dev)
    descale = one.expand(B, H)  # what fp8_kv.unit_descale hands the reference's call
    a = attention.flash_attn_varlen_func(
        q=q, k=fd[:, 0], v=fd[:, 1], max_seqlen_q=1, cu_seqlens_q=torch.arange(B + 1, dtype=torch.int32, device=dev),
        max_seqlen_k=None, seqused_k=lens, block_table=bt, softmax_scale=0.1, causal=True, fa_version=3,
        q_descale=descale, k_descale=descale, v_descale=descale)
    b = attention.paged_decode_attention(q, fd[:, 0], fd[:, 1], bt, lens, 0.1)
    assert torch.equal(a, b)
    with pytest.raises(AssertionError):  # no cu_seqlens_q
        attention.flash_attn_varlen_func(q, fd[:, 0], fd[:, 1], 2, None, seqused_k=lens, block_table=bt)
    # 32 heads over one kv head: past the decode reader's 16 rows, the prefill kernel reads it
    q32 = q.to(torch.float32).repeat(1, 8, 1)[:, :32].to(torch.bfloat16)
    c = attention.flash_attn_varlen_func(q32, fd[:, 0, :, :1], fd[:, 1, :, :1], 1,
                                         torch.arange(B + 1, dtype=torch.int32, device=dev), seqused_k=lens,
                                         block_table=bt, softmax_scale=0.1, causal=True)
    d = attention.paged_prefill_attention(q32, fd[:, 0, :, :1], fd[:, 1, :, :1], bt, lens, None, 1, 0.1)
    assert torch.equal(c, d)


@pytest.mark.parametrize("Hq,Hkv,length", [(8, 2, 20000), (64, 8, 9000), (3, 1, 33000)])
def test_single_long_sequence_combine_waves(dev, Hq, Hkv, length):
    """One sequence spread over every run of the balanced schedule: hundreds of
    records per (sequence, kv head), merged by several combine waves per query
    head (up to 1024 threads for groups of 8)."""
    P = -(-length // 16) + 8
    _case(dev, 61 + Hkv, 1, Hq, Hkv, 16, P, [length], "bf16", torch.float32, "per_seq_head")


@pytest.mark.parametrize("seed", range(12))
def test_decode_attention_random_shapes(dev, seed):
    """Seeded random batches for the matrix-core P V path: group sizes 1-8,
    power-of-two pages 16-64 (the ring kernels), 1-40 sequences (per-head and
    head-parallel schedules, and the split schedule on every third case),
    lengths 0-3000 with ragged last tiles, fp8 and bf16 queries, descales."""
    rng = np.random.default_rng(1000 + seed)
    G = int(rng.integers(1, 9))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    ps = int(rng.choice([16, 32, 64]))
    B = int(rng.choice([1, 2, 3, 7, 8, 13, 40]))
    lens = rng.integers(0, 3000, B).tolist()
    lens[int(rng.integers(0, B))] = int(rng.integers(1, 3000))  # at least one non-empty sequence
    P = max(64, sum(-(-x // ps) for x in lens) + 8)
    q_dtype = "fp8" if seed % 2 else "bf16"
    out_dtype = torch.float32 if seed % 4 < 2 else torch.bfloat16
    descales = [None, "scalar", "per_seq_head"][seed % 3]
    num_splits = 0 if seed % 3 else int(rng.integers(1, 24))
    print(f"random {seed}: G={G} Hkv={Hkv} ps={ps} B={B} splits={num_splits} {q_dtype}", flush=True)
    _case(dev, 2000 + seed, B, G * Hkv, Hkv, ps, P, lens, q_dtype, out_dtype, descales, num_splits=num_splits)


@pytest.mark.parametrize("seed", range(8))
def test_decode_attention_random_general_pages(dev, seed):
    """Seeded random batches on pages that are not a power of two >= 16 (1 to
    100 tokens): the general-page variants of every schedule, with the same
    groups, lengths, dtypes and descales as the power-of-two cases."""
    rng = np.random.default_rng(3000 + seed)
    G = int(rng.integers(1, 9))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    ps = int(rng.choice([1, 3, 8, 12, 24, 40, 100]))
    B = int(rng.choice([1, 2, 3, 7, 8, 13, 40]))
    lens = rng.integers(0, 3000, B).tolist()
    lens[int(rng.integers(0, B))] = int(rng.integers(1, 3000))
    P = max(64, sum(-(-x // ps) for x in lens) + 8)
    q_dtype = "fp8" if seed % 2 else "bf16"
    out_dtype = torch.float32 if seed % 4 < 2 else torch.bfloat16
    descales = [None, "scalar", "per_seq_head"][seed % 3]
    num_splits = 0 if seed % 3 else int(rng.integers(1, 24))
    print(f"random general {seed}: G={G} Hkv={Hkv} ps={ps} B={B} splits={num_splits} {q_dtype}", flush=True)
    _case(dev, 4000 + seed, B, G * Hkv, Hkv, ps, P, lens, q_dtype, out_dtype, descales, num_splits=num_splits)
