"""Paged decode attention over the FP8 KV cache: the reader of what the append
writes.

The reference decodes an FP8 cache through vLLM's FA3 fork,
``flash_attn_varlen_func(q=quantize(query), k, v, max_seqlen_q,
cu_seqlens_q, max_seqlen_k=None, seqused_k, block_table, softmax_scale,
causal, fa_version=3, q_descale, k_descale, v_descale)``
(pipeswift/llms/layers/attention.py:148-187), with every descale 1.0
(pipeswift/utils/fp8_kv.py:94-103).  ``flash_attn_varlen_func`` here takes the
same arguments for decode and speculative decode (a few query tokens per
sequence, causal with FA's bottom-right alignment) and runs
``psk_paged_decode_attention``: Q K^T on the bf16 MFMA over exactly converted
FP8 values (gfx950's FP8 MFMA truncates its sums), fp32 softmax, P V on the
bf16 MFMA with P split into hi + lo bf16 parts (2^-17 relative per weight,
fp32 sums) for every block size, and descales of any value per (sequence,
kv head) -- for instance the per-tensor
scales ``cache_ops.compute_kv_scales`` gave the append.

The query tokens of a sequence and the query heads of a kv head share the
16 rows of one MFMA tile of the decode reader: ``max_seqlen_q * Hq / Hkv`` at
most 16 (e.g. 4 draft positions at 4 heads per kv head).  Larger steps --
prefill and chunked prefill, which the reference sends through the same entry
-- run ``psk_paged_prefill_attention`` (``paged_prefill_attention``): the same
arithmetic, with each kv head's keys read once per 256 query rows.
"""

from __future__ import annotations

import os
from typing import Optional

import torch

from ._lib import check, dtype_code, i64_array, lib, ptr, stream_handle

HEAD_DIM = 128
MAX_ROWS = 16  # query tokens x query heads per kv head
# Opt-in argument checks that need a host synchronization (check_cu_seqlens_q).
_CHECK_ARGS = os.environ.get("PIPESWIFT_AMD_CHECK_ARGS", "0") == "1"

_OUT_CODES = {torch.bfloat16: 2, torch.float32: 0}


def workspace_floats(num_seqs: int, num_q_heads: int, num_kv_heads: int, max_seq_len: int, num_splits: int = 0,
                     q_len: int = 1) -> int:
    n = int(lib().psk_paged_decode_workspace_len(num_seqs, q_len, num_q_heads, num_kv_heads, max_seq_len,
                                                  num_splits))
    if n < 0:
        check(n, "paged decode workspace")
    return n


def _descale(t: Optional[torch.Tensor], num_seqs: int, num_kv_heads: int, device):
    """(device pointer, stride over sequences, stride over kv heads) of a
    descale given as None, a one-element tensor, or a (num_seqs, num_kv_heads)
    tensor (stride-0 expansions included, as vLLM passes them)."""
    if t is None:
        return None, 0, 0
    assert t.dtype == torch.float32 and t.device == device, "descales are float32 tensors on the query's device"
    if t.numel() == 1:
        return t, 0, 0
    assert t.dim() == 2 and t.shape[0] >= num_seqs and t.shape[1] == num_kv_heads, \
        f"descale shape {tuple(t.shape)}, want ({num_seqs}, {num_kv_heads})"
    return t, t.stride(0), t.stride(1)


def check_cu_seqlens_q(cu_seqlens_q: torch.Tensor, total_q: int, q_len: int) -> None:
    """Validate a ragged query layout against what the reader assumes (an
    AssertionError naming the first violation): ``cu_seqlens_q`` is int32
    [B + 1], starts at 0, never decreases, ends at most at ``total_q`` (the
    query rows), and gives no sequence more than ``q_len`` rows.  The reader
    itself trusts the layout: a longer sequence is cut to its first ``q_len``
    rows (the others of a fresh output stay unwritten), and an end past
    ``total_q`` writes output rows past the tensor.  This check copies the
    array to the host (a synchronization), so it is opt-in."""
    cu = cu_seqlens_q.detach().to("cpu", torch.int64)
    assert cu.dim() == 1 and cu.numel() >= 1, f"cu_seqlens_q must be 1-D [B + 1], got shape {tuple(cu.shape)}"
    assert int(cu[0]) == 0, f"cu_seqlens_q[0] = {int(cu[0])}, must be 0"
    n = cu[1:] - cu[:-1]
    if n.numel():
        b = int(torch.argmin(n))
        assert int(n[b]) >= 0, f"cu_seqlens_q decreases at sequence {b}: {int(cu[b])} -> {int(cu[b + 1])}"
        b = int(torch.argmax(n))
        assert int(n[b]) <= q_len, f"sequence {b} has {int(n[b])} query rows, more than max_seqlen_q = {q_len}"
    assert int(cu[-1]) <= total_q, f"cu_seqlens_q[-1] = {int(cu[-1])} exceeds the {total_q} query rows"


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    softmax_scale: Optional[float] = None,
    q_descale: Optional[torch.Tensor] = None,
    k_descale: Optional[torch.Tensor] = None,
    v_descale: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    return_softmax_lse: bool = False,
    max_seq_len: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
    num_splits: int = 0,
    q_len: int = 1,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    causal: bool = True,
    validate: bool = False,
):
    """One decode step of attention for every sequence.

    q: [total_q, Hq, 128] (fp8 e4m3fn used as is; bf16/fp16/fp32 quantized as
    e4m3(q / q_descale), as the reference quantizes its query).  Sequence b
    owns query rows [cu_seqlens_q[b], cu_seqlens_q[b+1]) (int32 [B+1]; None:
    q_len rows each, total_q = B * q_len), at most ``q_len`` of them: its last
    positions.  With ``causal`` query token i of n sees the first
    seq_lens[b] - n + 1 + i keys (FA's bottom-right alignment), else all.
    k_cache, v_cache: fp8 [num_blocks, block_size, Hkv, 128] (views of the fused
    [P, 2, ps, H, D] layer are fine).  block_table: int32 [B, W];
    seq_lens: int32 [B] (``seqused_k``).  Returns out [total_q, Hq, 128] (bf16
    unless ``out`` is given as float32) and, when asked, lse [Hq, total_q]
    float32; rows no sequence owns are left as they were.
    ``num_splits``: workgroups per longest sequence, as FA's; 0 (default)
    balances the work instead: one workgroup per resident slot, each streaming
    an equal run of the batch's 16-token tiles of one kv head across sequence
    boundaries.

    Contract of a ragged ``cu_seqlens_q`` (not checked on the fast path):
    cu[-1] <= total_q and every sequence has at most ``q_len`` rows.
    ``validate=True`` (or PIPESWIFT_AMD_CHECK_ARGS=1) checks it with a host
    synchronization first (``check_cu_seqlens_q``); the check is skipped while
    the stream is being captured into a graph.
    """
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda
    assert q.dim() == 3 and q.shape[2] == HEAD_DIM and q.stride(2) == 1, "q must be [B, Hq, 128] with unit last stride"
    assert k_cache.dtype == torch.float8_e4m3fn and v_cache.dtype == torch.float8_e4m3fn, "the cache must be fp8 e4m3fn"
    assert k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.shape[3] == HEAD_DIM
    assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1
    TQ, Hq, _ = q.shape
    P, ps, Hkv, _ = k_cache.shape
    q_len = int(q_len)
    assert q_len >= 1
    if cu_seqlens_q is None:
        assert TQ % q_len == 0, f"{TQ} query rows are not {q_len} per sequence"
        B = TQ // q_len
    else:
        assert cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.is_contiguous() and cu_seqlens_q.dim() == 1
        assert cu_seqlens_q.device == q.device
        B = cu_seqlens_q.shape[0] - 1
        if (validate or _CHECK_ARGS) and not torch.cuda.is_current_stream_capturing():
            check_cu_seqlens_q(cu_seqlens_q, TQ, q_len)
    assert Hq % Hkv == 0 and q_len * (Hq // Hkv) <= MAX_ROWS, \
        f"{q_len} query tokens x {Hq // Hkv} heads per kv head (at most {MAX_ROWS} rows)"
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.stride(1) == 1
    assert block_table.shape[0] >= B
    assert seq_lens.dtype == torch.int32 and seq_lens.is_contiguous() and seq_lens.numel() >= B
    device = q.device
    if softmax_scale is None:
        softmax_scale = HEAD_DIM ** -0.5
    if max_seq_len is None:
        max_seq_len = block_table.shape[1] * ps  # bounds every sequence, no host sync
    if out is None:
        out = torch.empty(TQ, Hq, HEAD_DIM, dtype=torch.bfloat16, device=device)
    assert out.dtype in _OUT_CODES and out.shape == (TQ, Hq, HEAD_DIM) and out.stride(2) == 1
    lse = torch.empty(Hq, TQ, dtype=torch.float32, device=device) if return_softmax_lse else None
    need = workspace_floats(B, Hq, Hkv, max_seq_len, num_splits, q_len)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.float32, device=device)
    qd, qsb, qsh = _descale(q_descale, B, Hkv, device)
    kd, ksb, ksh = _descale(k_descale, B, Hkv, device)
    vd, vsb, vsh = _descale(v_descale, B, Hkv, device)
    st = lib().psk_paged_decode_attention(
        q.data_ptr(), q.stride(0), q.stride(1), dtype_code(q.dtype),
        k_cache.data_ptr(), v_cache.data_ptr(), i64_array(k_cache.stride()[:3]), i64_array(v_cache.stride()[:3]),
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(), B, Hq, Hkv,
        HEAD_DIM, ps, P, int(max_seq_len), int(num_splits), q_len, ptr(cu_seqlens_q), 1 if causal else 0,
        float(softmax_scale), ptr(qd), ptr(kd), ptr(vd),
        i64_array([qsb, qsh, ksb, ksh, vsb, vsh]), out.data_ptr(), out.stride(0), out.stride(1),
        _OUT_CODES[out.dtype], ptr(lse), TQ if lse is not None else 0, workspace.data_ptr(), workspace.numel(),
        stream_handle(device),
    )
    check(st, "paged_decode_attention")
    return (out, lse) if return_softmax_lse else out


def prefill_workspace_words(num_seqs: int) -> int:
    n = int(lib().psk_paged_prefill_workspace_len(num_seqs))
    if n < 0:
        check(n, "paged prefill workspace")
    return n


def paged_prefill_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: Optional[torch.Tensor],
    max_seqlen_q: int,
    softmax_scale: Optional[float] = None,
    q_descale: Optional[torch.Tensor] = None,
    k_descale: Optional[torch.Tensor] = None,
    v_descale: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    return_softmax_lse: bool = False,
    causal: bool = True,
    workspace: Optional[torch.Tensor] = None,
    validate: bool = False,
):
    """Attention of a prefill (or chunked-prefill) step over the paged FP8
    cache: ``paged_decode_attention``'s arguments and results (q~, scores,
    descales, FA's bottom-right causal rule, zero rows for missing pages, bf16
    or float32 ``out``, lse [Hq, total_q]) for any number of query tokens per
    sequence, at most ``max_seqlen_q`` each, and up to 256 query heads per kv
    head.  One workgroup per (kv head, block of 256 / (Hq / Hkv) query tokens
    of one sequence) streams the sequence's keys once for the whole block
    through LDS; Q K^T runs on the bf16 MFMA over exactly converted FP8
    values and P V on the fp16 MFMA with V exact and P rounded once to fp16
    (at most (2^-11 + K 2^-25) max|V vd| more error for K keys), fp32 sums.
    ``workspace``: int32 of at
    least ``prefill_workspace_words(B)`` (allocated when absent).  The ragged
    layout contract, and ``validate``, are ``paged_decode_attention``'s."""
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda
    assert q.dim() == 3 and q.shape[2] == HEAD_DIM and q.stride(2) == 1, "q must be [T, Hq, 128] with unit last stride"
    assert k_cache.dtype == torch.float8_e4m3fn and v_cache.dtype == torch.float8_e4m3fn, "the cache must be fp8 e4m3fn"
    assert k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.shape[3] == HEAD_DIM
    assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1
    TQ, Hq, _ = q.shape
    P, ps, Hkv, _ = k_cache.shape
    q_len = int(max_seqlen_q)
    assert q_len >= 1
    if cu_seqlens_q is None:
        assert TQ % q_len == 0, f"{TQ} query rows are not {q_len} per sequence"
        B = TQ // q_len
    else:
        assert cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.is_contiguous() and cu_seqlens_q.dim() == 1
        assert cu_seqlens_q.device == q.device
        B = cu_seqlens_q.shape[0] - 1
        if (validate or _CHECK_ARGS) and not torch.cuda.is_current_stream_capturing():
            check_cu_seqlens_q(cu_seqlens_q, TQ, q_len)
    assert Hkv > 0 and Hq % Hkv == 0, f"{Hq} query heads over {Hkv} kv heads"
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.stride(1) == 1
    assert block_table.shape[0] >= B
    assert seq_lens.dtype == torch.int32 and seq_lens.is_contiguous() and seq_lens.numel() >= B
    device = q.device
    if softmax_scale is None:
        softmax_scale = HEAD_DIM ** -0.5
    if out is None:
        out = torch.empty(TQ, Hq, HEAD_DIM, dtype=torch.bfloat16, device=device)
    assert out.dtype in _OUT_CODES and out.shape == (TQ, Hq, HEAD_DIM) and out.stride(2) == 1
    lse = torch.empty(Hq, TQ, dtype=torch.float32, device=device) if return_softmax_lse else None
    need = prefill_workspace_words(B)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.int32, device=device)
    assert workspace.dtype == torch.int32 and workspace.device == device
    qd, qsb, qsh = _descale(q_descale, B, Hkv, device)
    kd, ksb, ksh = _descale(k_descale, B, Hkv, device)
    vd, vsb, vsh = _descale(v_descale, B, Hkv, device)
    st = lib().psk_paged_prefill_attention(
        q.data_ptr(), q.stride(0), q.stride(1), dtype_code(q.dtype),
        k_cache.data_ptr(), v_cache.data_ptr(), i64_array(k_cache.stride()[:3]), i64_array(v_cache.stride()[:3]),
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(), B, Hq, Hkv,
        HEAD_DIM, ps, P, TQ, q_len, ptr(cu_seqlens_q), 1 if causal else 0, float(softmax_scale),
        ptr(qd), ptr(kd), ptr(vd), i64_array([qsb, qsh, ksb, ksh, vsb, vsh]), out.data_ptr(), out.stride(0),
        out.stride(1), _OUT_CODES[out.dtype], ptr(lse), TQ if lse is not None else 0, workspace.data_ptr(),
        workspace.numel(), stream_handle(device),
    )
    check(st, "paged_prefill_attention")
    return (out, lse) if return_softmax_lse else out


def _chunked_queries(cu_seqlens_q, total_q, seqused_k, block_table, chunk, causal, descales):
    """Query tokens of each sequence cut into chunks of at most ``chunk``
    consecutive tokens, each chunk a sequence of its own for the reader, built
    on the device (no host synchronization).

    Chunk j of sequence b covers its query tokens [j*chunk, i1), consecutive
    rows of q, so q and the output keep their layout.  Its key length is the
    sequence's length minus the sequence's tokens after the chunk when causal
    (the reader's bottom-right alignment then shows each token the keys up to
    its own position), else the whole sequence.  How many chunks there are
    depends on the lengths, so the layout has a fixed bound of
    ceil(total_q / chunk) + B chunk slots; slots past the last chunk have no
    query rows and no keys.  Returns (cu_seqlens_q, seq_lens, block_table,
    descales) of the chunk sequences."""
    dev = cu_seqlens_q.device
    B = seqused_k.shape[0]
    cu = cu_seqlens_q.to(torch.int64)
    n = cu[1:] - cu[:-1]
    chunks = (n + chunk - 1) // chunk
    ends = torch.cumsum(chunks, 0)
    V = (total_q + chunk - 1) // chunk + B
    v = torch.arange(V, device=dev)
    b = torch.searchsorted(ends, v, right=True).clamp_(max=B - 1)
    live = v < ends[-1]
    j = v - (ends[b] - chunks[b])
    i1 = torch.minimum((j + 1) * chunk, n[b])
    cu2 = torch.empty(V + 1, dtype=torch.int32, device=dev)
    cu2[:V] = torch.where(live, cu[b] + j * chunk, cu[-1]).to(torch.int32)
    cu2[V] = cu[-1].to(torch.int32)
    L = seqused_k.to(torch.int64)[b]
    lens = (L - n[b] + i1) if causal else L
    lens = torch.where(live, lens, torch.zeros_like(lens)).clamp_(min=0).to(torch.int32)
    bt = block_table.index_select(0, b)
    out = []
    for d in descales:
        out.append(d.index_select(0, b) if d is not None and d.dim() == 2 and d.numel() > 1 else d)
    return cu2, lens, bt, out


def chunked_prefill_attention(q, k, v, max_seqlen_q, cu_seqlens_q, seqused_k, block_table, softmax_scale=None,
                              causal=False, q_descale=None, k_descale=None, v_descale=None,
                              return_softmax_lse=False, out=None, num_splits=0):
    """A prefill step read by the decode reader instead of the prefill kernel:
    each sequence's query tokens cut into chunks of 16 / (Hq / Hkv) tokens,
    each read as a sequence of its own (``_chunked_queries``).  Exact, but
    every chunk streams its sequence's keys again, so a prefill of n tokens
    over L keys reads about n / chunk times the cache bytes of one pass; kept
    as an independent second path for cross-checks and as the prefill
    kernel's measured baseline.  At most 16 query heads per kv head."""
    group = q.shape[1] // k.shape[2]
    assert 1 <= group <= MAX_ROWS, f"{group} query heads per kv head: the decode reader takes at most {MAX_ROWS}"
    chunk = MAX_ROWS // group
    cu2, lens2, bt2, (qd, kd, vd) = _chunked_queries(cu_seqlens_q, q.shape[0], seqused_k, block_table, chunk,
                                                     causal, (q_descale, k_descale, v_descale))
    return paged_decode_attention(q, k, v, bt2, lens2, softmax_scale, qd, kd, vd, out=out,
                                  return_softmax_lse=return_softmax_lse, max_seq_len=block_table.shape[1] * k.shape[1],
                                  num_splits=num_splits, q_len=chunk, cu_seqlens_q=cu2, causal=causal)


def flash_attn_varlen_func(
    q,
    k,
    v,
    max_seqlen_q,
    cu_seqlens_q,
    max_seqlen_k=None,
    seqused_k=None,
    block_table=None,
    softmax_scale=None,
    causal=False,
    fa_version=3,
    q_descale=None,
    k_descale=None,
    v_descale=None,
    return_softmax_lse=False,
    out=None,
    num_splits=0,
):
    """The FA3 entry the reference's ``_fp8_paged_attn`` calls
    (attention.py:166-184) for decode, speculative decode and prefill: q is
    [total_q, Hq, D], sequence b's query tokens at rows
    [cu_seqlens_q[b], cu_seqlens_q[b+1]), at most ``max_seqlen_q`` of them,
    the sequence's last positions; with ``causal`` each sees the keys up to
    its own position.  ``max_seqlen_k`` bounds the lengths when given, else
    the block table's width does.  ``num_splits`` is the flash-decoding split
    count (0: the balanced schedule); ``fa_version`` is accepted for signature
    compatibility.

    A sequence's query tokens and the query heads of a kv head share the 16
    rows of one MFMA tile of the decode reader.  When ``max_seqlen_q * Hq /
    Hkv`` exceeds 16 (a prefill or chunked-prefill step, which the reference
    routes through this same entry, attention.py:577-585, or more than 16
    query heads per kv head) the step runs ``paged_prefill_attention``, which
    reads each kv head's keys once per block of 256 query rows; ``num_splits``
    and ``max_seqlen_k`` do not apply there."""
    assert seqused_k is not None and block_table is not None, "paged attention needs seqused_k and block_table"
    B = seqused_k.shape[0]
    assert cu_seqlens_q is not None and cu_seqlens_q.shape[0] == B + 1
    group = q.shape[1] // k.shape[2] if k.shape[2] else 0
    q_len = int(max_seqlen_q)
    ps = k.shape[1]
    bound = block_table.shape[1] * ps if max_seqlen_k is None else min(int(max_seqlen_k), block_table.shape[1] * ps)
    if q_len * max(group, 1) > MAX_ROWS:
        return paged_prefill_attention(q, k, v, block_table, seqused_k, cu_seqlens_q, q_len, softmax_scale,
                                       q_descale, k_descale, v_descale, out=out,
                                       return_softmax_lse=return_softmax_lse, causal=causal)
    # B rows of at most one token each: one per sequence, cu_seqlens_q is 0..B
    cu = None if q_len == 1 and q.shape[0] == B else cu_seqlens_q
    return paged_decode_attention(q, k, v, block_table, seqused_k, softmax_scale, q_descale, k_descale, v_descale,
                                  out=out, return_softmax_lse=return_softmax_lse, max_seq_len=bound,
                                  num_splits=num_splits, q_len=q_len, cu_seqlens_q=cu, causal=causal)
