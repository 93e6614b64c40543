"""Pins of the oracle's paged decode attention (oracle/kv_oracle.py) on the CPU:
torch's own scaled_dot_product_attention over a dense gather of the same pages
(float64, K/V heads repeated per query group), the reference's accuracy gate as a
closed form (a constant V comes back exactly; scripts/check_fp8_kv_backend.py),
a one-token sequence, the log-sum-exp, and page-permutation invariance; with
several query tokens per sequence, torch SDPA under torch's bottom-right causal
mask, and the reduction of each causal token to one-token decode."""

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O


def make_case(seed, B=3, Hq=8, Hkv=2, P=40, ps=16, max_len=200, q_dtype="bf16"):
    rng = np.random.default_rng(seed)
    k = (rng.standard_normal((P, ps, Hkv, 128)) * 2).astype(np.float32)
    v = (rng.standard_normal((P, ps, Hkv, 128)) * 2).astype(np.float32)
    kc = torch.from_numpy(k).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    vc = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    lens = rng.integers(1, max_len, B)
    W = int(-(-lens.max() // ps))
    bt = np.stack([rng.permutation(P)[:W] for _ in range(B)]).astype(np.int32)
    qf = (rng.standard_normal((B, Hq, 128)) * 3).astype(np.float32)
    q = torch.from_numpy(qf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return q, kc, vc, bt, lens


def sdpa_reference(q, kc, vc, bt, lens, scale, qd, kd, vd):
    """torch SDPA in float64 over densely gathered pages; q quantized with torch's
    own float8 conversion."""
    B, Hq, D = q.shape
    _, ps, Hkv, _ = kc.shape
    G = Hq // Hkv
    k8 = torch.from_numpy(kc).view(torch.float8_e4m3fn).double()
    v8 = torch.from_numpy(vc).view(torch.float8_e4m3fn).double()
    qb = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).float()
    out = torch.zeros(B, Hq, D, dtype=torch.float64)
    for b in range(B):
        n = int(lens[b])
        idx = torch.arange(n)
        pages = torch.from_numpy(bt[b].astype(np.int64))[idx // ps]
        K = k8[pages, idx % ps]  # [n, Hkv, D]
        V = v8[pages, idx % ps]
        qdb = torch.tensor(qd[b], dtype=torch.float32).repeat_interleave(G)[:, None]
        qq = ((qb[b] / qdb).clamp(-448, 448).to(torch.float8_e4m3fn)).double()  # [Hq, D]
        Kr = K.repeat_interleave(G, dim=1).permute(1, 0, 2)  # [Hq, n, D]
        Vr = V.repeat_interleave(G, dim=1).permute(1, 0, 2)
        sc = float(scale) * (torch.from_numpy(qd[b]).double() * torch.from_numpy(kd[b]).double()).repeat_interleave(G)
        o = torch.stack([torch.nn.functional.scaled_dot_product_attention(
            qq[hq][None, None], Kr[hq][None], Vr[hq][None], scale=float(sc[hq]))[0, 0] for hq in range(Hq)])
        out[b] = o * torch.from_numpy(vd[b]).double().repeat_interleave(G)[:, None]
    return out.numpy()


@pytest.mark.parametrize("seed,Hq,Hkv,ps", [(0, 8, 2, 16), (1, 4, 4, 8), (2, 8, 1, 32), (3, 10, 2, 16)])
def test_oracle_matches_torch_sdpa(seed, Hq, Hkv, ps):
    q, kc, vc, bt, lens = make_case(seed, Hq=Hq, Hkv=Hkv, ps=ps)
    rng = np.random.default_rng(seed + 100)
    B = q.shape[0]
    qd, kd, vd = [rng.uniform(0.5, 2.0, (B, Hkv)).astype(np.float32) for _ in range(3)]
    scale = 0.0883883
    got, lse = O.paged_decode_attention(q, "bf16", kc, vc, bt, lens, scale, qd, kd, vd)
    exp = sdpa_reference(q, kc, vc, bt, lens, np.float32(scale), qd, kd, vd)
    np.testing.assert_allclose(got, exp, rtol=1e-10, atol=1e-10)


def test_constant_values_come_back_exactly():
    """scripts/check_fp8_kv_backend.py: V constant per kv head -> out == V."""
    rng = np.random.default_rng(9)
    P, ps, Hkv, Hq = 64, 64, 4, 32
    k = torch.from_numpy(rng.standard_normal((P, ps, Hkv, 128)).astype(np.float32)).to(torch.float8_e4m3fn)
    vals = np.array([1.0, 1.5, 2.0, 3.0], dtype=np.float32)
    v = torch.from_numpy(np.broadcast_to(vals[None, None, :, None], (P, ps, Hkv, 128)).copy()).to(torch.float8_e4m3fn)
    q = torch.from_numpy(rng.standard_normal((1, Hq, 128)).astype(np.float32)).to(torch.float8_e4m3fn)
    bt = np.arange(P, dtype=np.int32)[None]
    out, _ = O.paged_decode_attention(q.view(torch.uint8).numpy(), "fp8", k.view(torch.uint8).numpy(),
                                      v.view(torch.uint8).numpy(), bt, [P * ps], 128 ** -0.5)
    exact = np.repeat(vals, Hq // Hkv)[:, None]
    assert np.abs(out[0] / exact - 1).max() < 1e-12


def test_one_token_lse_and_empty_sequence():
    q, kc, vc, bt, _ = make_case(5, B=2, Hq=4, Hkv=2)
    out, lse = O.paged_decode_attention(q, "bf16", kc, vc, bt, [1, 0], 0.1, None, None, None)
    v0 = O.e4m3fn_to_f32(vc[bt[0, 0], 0]).astype(np.float64)  # [Hkv, D]
    np.testing.assert_array_equal(out[0], np.repeat(v0, 2, axis=0))
    assert (out[1] == 0).all() and np.isneginf(lse[1]).all()
    # lse of a longer sequence against torch.logsumexp of the scores
    q, kc, vc, bt, lens = make_case(6, B=1, Hq=2, Hkv=1, max_len=120)
    out, lse = O.paged_decode_attention(q, "bf16", kc, vc, bt, lens, 0.125)
    n, ps = int(lens[0]), kc.shape[1]
    idx = np.arange(n)
    K = O.e4m3fn_to_f32(kc[bt[0, idx // ps], idx % ps, 0]).astype(np.float64)
    qq = O.e4m3fn_to_f32(O.quantize_e4m3(O.to_f32(q[0], "bf16"))).astype(np.float64)
    s = torch.from_numpy(qq @ K.T * 0.125)
    np.testing.assert_allclose(lse[0], torch.logsumexp(s, dim=1).numpy(), rtol=1e-12)


def test_page_permutation_invariance():
    q, kc, vc, bt, lens = make_case(7, B=2, P=30)
    perm = np.random.default_rng(1).permutation(30)
    inv = np.argsort(perm)
    a, _ = O.paged_decode_attention(q, "bf16", kc, vc, bt, lens, 0.1)
    b, _ = O.paged_decode_attention(q, "bf16", kc[inv], vc[inv], perm[bt].astype(np.int32), lens, 0.1)
    np.testing.assert_array_equal(a, b)


def test_multi_token_causal_matches_torch_lower_right_sdpa():
    """Several query tokens per sequence (speculative decode), ragged counts:
    the oracle against torch SDPA under torch's own bottom-right causal mask
    (torch.nn.attention.bias.causal_lower_right), float64 over a dense gather;
    and without causal, against SDPA with no mask."""
    from torch.nn.attention.bias import causal_lower_right

    rng = np.random.default_rng(31)
    Hq, Hkv, P, ps = 8, 2, 60, 16
    G = Hq // Hkv
    counts = np.array([1, 3, 2, 4, 4])
    lens = np.array([5, 3, 40, 200, 1])  # a sequence shorter than its query count
    cu = np.concatenate([[0], np.cumsum(counts)])
    TQ = int(cu[-1])
    k = torch.from_numpy((rng.standard_normal((P, ps, Hkv, 128)) * 2).astype(np.float32)).to(torch.float8_e4m3fn)
    v = torch.from_numpy((rng.standard_normal((P, ps, Hkv, 128)) * 2).astype(np.float32)).to(torch.float8_e4m3fn)
    W = int(-(-lens.max() // ps))
    bt = np.stack([rng.permutation(P)[:W] for _ in range(len(lens))]).astype(np.int32)
    q8 = torch.from_numpy((rng.standard_normal((TQ, Hq, 128)) * 3).astype(np.float32)).to(torch.float8_e4m3fn)
    scale = float(np.float32(0.1))  # the kernel takes the scale as a float
    for causal in (True, False):
        got, lse = O.paged_decode_attention(q8.view(torch.uint8).numpy(), "fp8", k.view(torch.uint8).numpy(),
                                            v.view(torch.uint8).numpy(), bt, lens, scale, cu_seqlens_q=cu,
                                            causal=causal)
        for b in range(len(lens)):
            n, nq, c0 = int(lens[b]), int(counts[b]), int(cu[b])
            idx = torch.arange(n)
            pages = torch.from_numpy(bt[b].astype(np.int64))[idx // ps]
            K = k.double()[pages, idx % ps].repeat_interleave(G, dim=1).permute(1, 0, 2)[None]  # [1, Hq, n, D]
            V = v.double()[pages, idx % ps].repeat_interleave(G, dim=1).permute(1, 0, 2)[None]
            Q = q8.double()[c0:c0 + nq].permute(1, 0, 2)[None]  # [1, Hq, nq, D]
            if causal:
                mask = causal_lower_right(nq, n)._materialize()
                seen = mask.any(dim=1)  # tokens that see at least one key
                ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=scale)
                ref = torch.where(seen[None, None, :, None], ref, torch.zeros_like(ref))
                s = (Q @ K.transpose(-1, -2)) * scale
                ref_lse = torch.logsumexp(s.masked_fill(~mask, -float("inf")), dim=-1)
            else:
                ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=scale)
                ref_lse = torch.logsumexp((Q @ K.transpose(-1, -2)) * scale, dim=-1)
            np.testing.assert_allclose(got[c0:c0 + nq], ref[0].permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-10)
            exp_lse = ref_lse[0].T.numpy()
            np.testing.assert_allclose(lse[c0:c0 + nq], exp_lse, rtol=1e-12)


def test_multi_token_reduces_to_single_token_decode():
    """Causal query token i of n over a sequence of length L is the one-token
    decode of the same query over the first L - n + 1 + i keys: the last token
    is plain decode, earlier ones see a shorter sequence."""
    q, kc, vc, bt, _ = make_case(12, B=1, Hq=8, Hkv=2, max_len=300)
    rng = np.random.default_rng(3)
    nq, L = 4, bt.shape[1] * kc.shape[1] - 5
    qm = (rng.standard_normal((nq, 8, 128)) * 3).astype(np.float32)
    qm = torch.from_numpy(qm).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    qd, kd, vd = [rng.uniform(0.5, 2.0, (1, 2)).astype(np.float32) for _ in range(3)]
    got, lse = O.paged_decode_attention(qm, "bf16", kc, vc, bt, [L], 0.09, qd, kd, vd,
                                        cu_seqlens_q=[0, nq], causal=True)
    for i in range(nq):
        one, one_lse = O.paged_decode_attention(qm[i:i + 1], "bf16", kc, vc, bt, [L - nq + 1 + i], 0.09, qd, kd, vd)
        np.testing.assert_array_equal(got[i], one[0])
        np.testing.assert_array_equal(lse[i], one_lse[0])
