"""Host-side logic of the path, on the CPU: slot mapping / page table builder,
graph metadata refresh, the CopyEngine's coalescing and range check, and the
shims' argument checks that fire before any device call."""

from array import array

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd import metadata
from pipeswift_amd.copy_engine import coalesce_runs, page_bytes, validate_pages


class Seq:
    def __init__(self, seq_id, n_tokens, offset):
        self.seq_id = seq_id
        self.token_ids = list(range(n_tokens))
        self.offset = offset


@pytest.mark.parametrize("dcp,il", [(1, 1), (2, 1), (2, 8), (4, 4)])
def test_prepare_kv_info_matches_oracle(dcp, il):
    rng = np.random.default_rng(dcp * 7 + il)
    ps = 16
    seqs = [Seq(3, 100, 0), Seq(7, 45, 33), Seq(9, 17, 16), Seq(11, 64, 63)]
    table = {s.seq_id: rng.permutation(500)[: (len(s.token_ids) + ps - 1) // ps + 1].tolist() for s in seqs}
    for rank in range(dcp):
        info = metadata.prepare_kv_info(seqs, table, ps, None, None, dcp_interleave_size=il, dcp_deg=dcp,
                                        dcp_rank=rank, device="cpu")
        exp = np.concatenate([O.slot_mapping(table[s.seq_id], s.offset, len(s.token_ids), ps, dcp, rank, il)
                              for s in seqs])
        assert info.slot_mapping.dtype == torch.int64
        assert np.array_equal(info.slot_mapping.numpy(), exp)
        W = max(len(v) for v in table.values())
        assert info.page_table.shape == (4, W) and info.page_table.dtype == torch.int32
        for i, s in enumerate(seqs):
            row = info.page_table[i].numpy()
            assert list(row[: len(table[s.seq_id])]) == table[s.seq_id] and not row[len(table[s.seq_id]):].any()
        q = [len(s.token_ids) - s.offset for s in seqs]
        assert info.actual_lens_q.tolist() == q
        assert info.cu_seqlens_q.tolist() == [0] + list(np.cumsum(q))
        kv = [len(s.token_ids) if dcp == 1 else O.dcp_kv_len(s.offset, dcp, rank, il) for s in seqs]
        assert info.actual_lens_kv.tolist() == kv


def test_prepare_kv_info_page_table_containers_and_errors():
    from array import array

    ps = 16
    seqs = [Seq(1, 40, 0), Seq(2, 20, 19), Seq(3, 33, 32)]
    rows = {1: [7, 3, 9], 2: [4, 8], 3: [1, 2, 5]}
    exp = np.concatenate([O.slot_mapping(rows[s.seq_id], s.offset, len(s.token_ids), ps) for s in seqs])
    for make in (lambda r: array("i", r), list, lambda r: np.array(r, np.int64), lambda r: torch.tensor(r)):
        info = metadata.prepare_kv_info(seqs, {k: make(v) for k, v in rows.items()}, ps, None, None, device="cpu")
        assert np.array_equal(info.slot_mapping.numpy(), exp)
        assert info.page_table.tolist() == [[7, 3, 9], [4, 8, 0], [1, 2, 5]]
    with pytest.raises(IndexError, match="needs page 2 of 2"):
        metadata.prepare_kv_info([Seq(2, 33, 30)], rows, ps, None, None, device="cpu")
    empty = metadata.prepare_kv_info([Seq(2, 20, 20)], rows, ps, None, None, device="cpu")
    assert empty.slot_mapping.numel() == 0 and empty.actual_lens_q.tolist() == [0]


def test_next_decode_step_metadata():
    ps = 16
    seqs = [Seq(0, 40, 39), Seq(1, 16, 15)]
    table = {0: [5, 9, 2, 7], 1: [4, 8]}
    info = metadata.prepare_kv_info(seqs, table, ps, None, None, is_decode=True, device="cpu")
    for s in seqs:
        s.offset += 1
        s.token_ids.append(0)
    nxt = metadata.derive_kvcache_info_next_decode_step(info, seqs, table, ps, device="cpu")
    assert nxt.slot_mapping.tolist() == [2 * 16 + 8, 8 * 16 + 0]
    assert nxt.actual_lens_kv.tolist() == [41, 17]


def test_next_decode_step_keeps_the_previous_steps_longer_lens():
    """A draft step over the first sequences of a longer previous step: lens_kv
    keeps every previous entry and advances only the stepped ones, as the
    reference's copy of the whole previous array does (metadata.py:367-369),
    so it stays as long as the lens_q / cu_seqlens_q taken from that step."""
    ps = 16
    seqs = [Seq(0, 40, 39), Seq(1, 16, 15), Seq(2, 70, 69)]
    table = {0: [5, 9, 2, 7], 1: [4, 8], 2: [1, 3, 6, 10, 11]}
    info = metadata.prepare_kv_info(seqs, table, ps, None, None, is_decode=True, device="cpu")
    assert info.actual_lens_kv_cpu.tolist() == [40, 16, 70]
    stepped = seqs[:2]
    for s in stepped:
        s.offset += 1
        s.token_ids.append(0)
    nxt = metadata.derive_kvcache_info_next_decode_step(info, stepped, table, ps, device="cpu")
    assert nxt.slot_mapping.tolist() == [2 * 16 + 8, 8 * 16 + 0]
    assert nxt.actual_lens_kv_cpu.tolist() == [41, 17, 70] == nxt.actual_lens_kv.tolist()
    assert nxt.actual_lens_kv.shape[0] == nxt.actual_lens_q.shape[0] == nxt.cu_seqlens_q.shape[0] - 1


def test_graph_refresh_oracle_hand_worked():
    """The oracle of set_graph_kvcacheinfo (cudagraph.py:75-118) on a case
    worked out by hand: 2 live sequences in a graph of 4, static buffers of 5
    rows and 4 page columns, a 3-wide step page table, 2 tokens per sequence
    (pad_q_len 2)."""
    static = {"page_table": np.full((5, 4), 9, np.int32), "slot_mapping": np.full(10, 77, np.int64),
              "lens_q": np.full(5, 7, np.int32), "lens_kv": np.full(5, 7, np.int32),
              "cu_seqlens_q": np.full(6, 7, np.int32)}
    step = {"page_table": np.array([[1, 2, 3], [4, 5, 0]], np.int32), "slot_mapping": np.array([16, 17, 64, 65]),
            "lens_q": np.array([2, 2], np.int32), "lens_kv": np.array([40, 18], np.int32),
            "cu_seqlens_q": np.array([0, 2, 4], np.int32)}
    O.graph_refresh(static, step, cg_bsz=4, pad_q_len=2)
    assert static["page_table"].tolist() == [[1, 2, 3, 9], [4, 5, 0, 9], [0, 0, 0, 9], [0, 0, 0, 9], [0, 0, 0, 9]]
    assert static["slot_mapping"].tolist() == [16, 17, 64, 65, -1, -1, -1, -1, -1, -1]
    assert static["lens_q"].tolist() == [2, 2, 2, 2, 2]
    assert static["lens_kv"].tolist() == [40, 18, 0, 0, 0]
    assert static["cu_seqlens_q"].tolist() == [0, 2, 4, 6, 8, 10]
    # an unpadded refresh (bsz == cg_bsz) leaves everything past the batch alone
    static2 = {k: v.copy() for k, v in static.items()}
    step2 = {"page_table": np.array([[8, 8, 8]] * 4, np.int32), "slot_mapping": np.array([1, 2, 3, 4]),
             "lens_q": np.ones(4, np.int32), "lens_kv": np.full(4, 3, np.int32),
             "cu_seqlens_q": np.arange(5, dtype=np.int32)}
    O.graph_refresh(static2, step2, cg_bsz=4, pad_q_len=1)
    assert static2["page_table"][4].tolist() == [0, 0, 0, 9] and static2["slot_mapping"][4:].tolist() == [-1] * 6
    assert static2["lens_q"].tolist() == [1, 1, 1, 1, 2] and static2["cu_seqlens_q"].tolist() == [0, 1, 2, 3, 4, 10]


@pytest.mark.parametrize("dcp,il", [(1, 1), (2, 1), (2, 4), (4, 2)])
def test_next_decode_step_native_matches_oracle(dcp, il):
    rng = np.random.default_rng(dcp * 10 + il)
    ps = 16
    B = 37
    for rank in range(dcp):
        seqs, table, rows = [], {}, []
        for b in range(B):
            n = int(rng.integers(1, 300))
            pages = (n + ps - 1) // ps
            row = rng.permutation(5000)[:pages].astype(np.int32)
            table[b] = array("i", row.tolist()) if b % 2 else row.tolist()
            rows.append(row.tolist())
            seqs.append(Seq(b, n, n - 1))
        info = metadata.prepare_kv_info(seqs, table, ps, None, None, is_decode=True, dcp_deg=dcp, dcp_rank=rank,
                                        dcp_interleave_size=il, device="cpu")
        for s in seqs:
            s.offset = len(s.token_ids) - 1
        nxt = metadata.derive_kvcache_info_next_decode_step(info, seqs, table, ps, dcp_interleave_size=il,
                                                            dcp_deg=dcp, dcp_rank=rank, device="cpu")
        slots, lens = O.next_decode_step(rows, [s.offset for s in seqs], info.actual_lens_kv_cpu.tolist(), ps,
                                         dcp, rank, il)
        assert nxt.slot_mapping.tolist() == slots.tolist()
        assert nxt.actual_lens_kv.tolist() == lens.tolist() == nxt.actual_lens_kv_cpu.tolist()
        assert nxt.page_table is info.page_table and nxt.cu_seqlens_q is info.cu_seqlens_q


def test_next_decode_step_position_without_page():
    seqs = [Seq(0, 40, 39)]
    table = {0: [5, 9, 2]}
    info = metadata.prepare_kv_info(seqs, table, 16, None, None, is_decode=True, device="cpu")
    seqs[0].offset = 48  # page 3 of a 3-page table
    with pytest.raises(IndexError, match="needs page 3 of 3"):
        metadata.derive_kvcache_info_next_decode_step(info, seqs, table, 16, device="cpu")
    with pytest.raises(IndexError):
        O.next_decode_step([[5, 9, 2]], [48], [40], 16)


@pytest.mark.parametrize("seed", range(10))
def test_copy_engine_coalesce_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    src = rng.permutation(1000)[:n].astype(np.uint64)
    dst = (src + 3) if seed % 2 else rng.permutation(1000)[:n].astype(np.uint64)
    got = coalesce_runs(src, dst)
    exp = O.coalesce(src, dst)
    for a, b in zip(got, exp):
        assert np.array_equal(a, b)
    # runs cover every page once and preserve the pairing
    s, d, ln = got
    pairs = {(int(a) + i, int(b) + i) for a, b, k in zip(s, d, ln) for i in range(int(k))}
    assert pairs == {(int(a), int(b)) for a, b in zip(src, dst)}


def test_copy_engine_page_validation():
    with pytest.raises(AssertionError, match=r"L2 store source: 1 of 2 page ids are not pages of the gpu tier "
                                             r"\(it has 10\): 10$"):
        validate_pages(np.array([1, 10]), 10, "gpu", "L2 store source")
    with pytest.raises(AssertionError, match=r"2 of 3 page ids .* l2 tier \(it has 20\): -1, 50$"):
        validate_pages(np.array([-1, 0, 50]), 20, "l2", "L2 load source")
    long = np.arange(100, 120)
    with pytest.raises(AssertionError, match=r"20 of 20 .*: 100, 101, 102, 103, 104, 105, 106, 107, \.\.\.$"):
        validate_pages(long, 10, "gpu", "x")
    validate_pages(np.array([9, 0]), 10, "gpu", "ok")
    validate_pages(np.array([], dtype=np.int64), 0, "gpu", "empty")


def test_page_bytes_matches_oracle():
    a = torch.empty(3, 10, 2, 16, 8, 128, dtype=torch.bfloat16)
    b = torch.empty(2, 10, 64, 576, dtype=torch.float8_e4m3fn)
    assert page_bytes([a, b]) == O.page_bytes([(a.shape, 2), (b.shape, 1)]) == 3 * 65536 + 2 * 64 * 576


def test_shim_asserts_fire_before_device_calls():
    from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash, reshape_and_cache_flash_diffkv

    k = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    c = torch.zeros(2, 16, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):  # CPU tensors: the reference asserts is_cuda too
        reshape_and_cache_flash(k, k, c, c, torch.zeros(4, dtype=torch.int64))
    with pytest.raises(AssertionError):
        reshape_and_cache_flash(k.view(4, 1024)[None], k, c, c, torch.zeros(4, dtype=torch.int64))
    with pytest.raises(AssertionError):
        reshape_and_cache_flash_diffkv(k, k, torch.zeros(2, 16, 8, 100), torch.zeros(4, dtype=torch.int64))


def test_fp8_reader_routes_steps_by_rows_per_kv_head(monkeypatch):
    """The FA3-style entry sends a step whose query tokens x query heads per
    kv head fit the decode reader's 16 MFMA rows to paged_decode_attention
    (decode, speculative decode) and every larger one -- prefill, chunked
    prefill, groups of more than 16 heads -- to paged_prefill_attention, with
    the caller's arguments (host tensors: the calls are intercepted)."""
    from pipeswift_amd import attention, fp8_kv

    calls = []
    monkeypatch.setattr(attention, "paged_decode_attention", lambda *a, **k: calls.append(("decode", a, k)) or "d")
    monkeypatch.setattr(attention, "paged_prefill_attention", lambda *a, **k: calls.append(("prefill", a, k)) or "p")
    f = fp8_kv.attn_varlen_func()
    bt = torch.zeros(2, 8, dtype=torch.int32)
    lens = torch.full((2,), 100, dtype=torch.int32)
    cu = torch.tensor([0, 8, 16], dtype=torch.int32)
    for Hq, Hkv, q_len, want in [(32, 8, 4, "decode"), (32, 8, 5, "prefill"), (8, 8, 16, "decode"),
                                 (8, 8, 17, "prefill"), (64, 2, 1, "prefill"), (16, 1, 1, "decode")]:
        k = torch.zeros(10, 16, Hkv, 128, dtype=torch.float8_e4m3fn)
        q = torch.zeros(16, Hq, 128, dtype=torch.bfloat16)
        got = f(q=q, k=k, v=k, max_seqlen_q=q_len, cu_seqlens_q=cu, seqused_k=lens, block_table=bt, causal=True,
                softmax_scale=0.25)
        assert got == want[0], (Hq, Hkv, q_len)
        kind, args, kw = calls[-1]
        assert kind == want
        if kind == "prefill":
            assert args[5] is cu and args[6] == q_len and args[7] == 0.25 and kw["causal"] is True


def test_chunked_prefill_layout():
    """The chunk sequences a prefill is read as (attention._chunked_queries), on
    the host: rows, causal key lengths and table rows of every chunk, against a
    direct enumeration."""
    from pipeswift_amd.attention import _chunked_queries

    counts = [5, 0, 1, 9, 4]
    lens = [5 + 30, 3, 1 + 7, 9, 4 + 100]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    bt = torch.arange(5 * 3, dtype=torch.int32).view(5, 3)
    ds = torch.arange(10, dtype=torch.float32).view(5, 2)
    for causal in (True, False):
        cu2, lens2, bt2, (qd, kd, vd) = _chunked_queries(cu, 21, torch.tensor(lens, dtype=torch.int32), bt, 4,
                                                           causal, (ds, None, ds[:1, :1]))
        exp_rows, exp_lens, exp_b = [], [], []
        for b, (n, L) in enumerate(zip(counts, lens)):
            for i0 in range(0, n, 4):
                i1 = min(i0 + 4, n)
                exp_rows.append((int(cu[b]) + i0, int(cu[b]) + i1))
                exp_lens.append(L - n + i1 if causal else L)
                exp_b.append(b)
        V = (21 + 3) // 4 + 5
        assert cu2.shape[0] == V + 1 and lens2.shape[0] == V and bt2.shape[0] == V
        k = len(exp_rows)
        assert [(int(cu2[i]), int(cu2[i + 1])) for i in range(k)] == exp_rows
        assert all(int(cu2[i]) == int(cu2[i + 1]) == 19 for i in range(k, V))  # empty slots at the end
        assert lens2[:k].tolist() == exp_lens and not lens2[k:].any()
        assert torch.equal(bt2[:k], bt[exp_b]) and torch.equal(qd[:k], ds[exp_b])
        assert kd is None and vd.shape == (1, 1)


def test_ragged_query_layout_check():
    """check_cu_seqlens_q, the reader's opt-in validation of a ragged query
    layout: each violation the reader would not survive is named."""
    from pipeswift_amd.attention import check_cu_seqlens_q

    ok = torch.tensor([0, 4, 5, 9], dtype=torch.int32)
    check_cu_seqlens_q(ok, 9, 4)
    check_cu_seqlens_q(ok, 12, 4)  # spare rows past the last sequence are allowed
    check_cu_seqlens_q(torch.tensor([0], dtype=torch.int32), 0, 1)
    with pytest.raises(AssertionError, match=r"sequence 2 has 5 query rows, more than max_seqlen_q = 4"):
        check_cu_seqlens_q(torch.tensor([0, 4, 5, 10], dtype=torch.int32), 10, 4)
    with pytest.raises(AssertionError, match=r"cu_seqlens_q\[-1\] = 9 exceeds the 8 query rows"):
        check_cu_seqlens_q(ok, 8, 4)
    with pytest.raises(AssertionError, match="decreases at sequence 1"):
        check_cu_seqlens_q(torch.tensor([0, 4, 3, 6], dtype=torch.int32), 8, 4)
    with pytest.raises(AssertionError, match=r"cu_seqlens_q\[0\] = 1"):
        check_cu_seqlens_q(torch.tensor([1, 4], dtype=torch.int32), 8, 4)
