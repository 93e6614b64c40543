"""numpy restatement of the reference's paged KV-cache semantics (test-only).

Tensors are numpy arrays holding raw element bits: bf16 and fp16 as uint16,
fp32 as uint32, fp8 E4M3FN as uint8.  ``dtype`` arguments are the strings
"bf16", "f16", "f32", "fp8".  Byte-copy semantics never look at the values;
only the FP8 paths convert to float32.

Reference files restated here (wsjdsg/PipeSwift):
  pipeswift/utils/triton_kernels/reshape_and_cache.py  (append, MLA concat, FP8)
  pipeswift/utils/fp8_kv.py:24-25,75-77                 (FP8 constants, quantize)
  pipeswift/utils/metadata.py:264-295, 351-414          (slot_mapping, page_table,
                                                         next decode step)
  pipeswift/utils/cudagraph.py:75-118                   (graph static refresh)
  pipeswift/utils/copy_engine.py:121-142, 373-427       (page bytes, views, range
                                                         check, run coalescing)
"""

from __future__ import annotations

import numpy as np

FP8_E4M3_MAX = 448.0  # fp8_kv.py:25, reshape_and_cache.py:8

RAW = {"bf16": np.uint16, "f16": np.uint16, "f32": np.uint32, "fp8": np.uint8}


# --------------------------------------------------------------------------- #
# element conversions
# --------------------------------------------------------------------------- #


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> float32 (exact: bf16 is the top half of an fp32)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0.

    Pinned against torch's ``Tensor.to(torch.bfloat16)`` on CPU.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r).astype(np.uint16)


def to_f32(raw: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_to_f32(raw)
    if dtype == "f16":
        return np.asarray(raw, dtype=np.uint16).view(np.float16).astype(np.float32)
    if dtype == "f32":
        raw = np.asarray(raw)
        return raw.view(np.float32) if raw.dtype == np.uint32 else raw.astype(np.float32)
    if dtype == "fp8":
        return e4m3fn_to_f32(raw)
    raise ValueError(dtype)


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_from_f32(x)
    if dtype == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)
    if dtype == "f32":
        return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    raise ValueError(dtype)


def e4m3fn_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> OCP E4M3FN byte, round to nearest even, NOT saturating.

    This is the plain dtype conversion ``Tensor.to(torch.float8_e4m3fn)``: a
    magnitude that rounds above 448 (anything above 464), inf and NaN all
    become the NaN code 0x7F with the input's sign.  The reference always
    clamps to +-448 first (reshape_and_cache.py:70-77, fp8_kv.py:75-77), so
    after the clamp only NaN reaches the NaN code.

    Method: for |x| >= 2^-6 (E4M3FN normals) drop 20 of fp32's 23 mantissa bits
    with round-half-even and rebias the exponent from 127 to 7; a mantissa
    carry rolls into the exponent by itself.  Below 2^-6 the code is
    round_half_even(|x| * 2^9), the count of 2^-9 subnormal steps (8 steps is
    the smallest normal, code 0x08).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mag = bits & np.uint32(0x7FFFFFFF)
    lsb = (mag >> 20) & 1
    rounded = (mag.astype(np.uint64) + 0x7FFFF + lsb) >> 20
    normal = rounded.astype(np.int64) - (120 << 3)  # (127 - 7) << 3
    with np.errstate(invalid="ignore", over="ignore"):
        sub = np.rint(np.abs(x) * np.float32(512.0))
    sub = np.where(mag < 0x3C800000, sub, 0).astype(np.int64)
    code = np.where(mag < 0x3C800000, sub, normal)
    code = np.where((mag >= 0x7F800000) | (code > 0x7E), 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


_E4M3_TABLE = None


def _e4m3_table() -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        b = np.arange(256, dtype=np.int64)
        s = np.where(b & 0x80, -1.0, 1.0)
        e = (b >> 3) & 0xF
        m = b & 7
        val = np.where(e == 0, np.ldexp(m.astype(np.float64), -9), np.ldexp(1.0 + m / 8.0, (e - 7).astype(np.int64)))
        val = s * val
        val[(e == 15) & (m == 7)] = np.nan
        _E4M3_TABLE = val.astype(np.float32)
    return _E4M3_TABLE


def e4m3fn_to_f32(q: np.ndarray) -> np.ndarray:
    """E4M3FN byte -> float32, exact; 0x7F/0xFF -> NaN.

    Pinned against torch's ``Tensor.view(torch.float8_e4m3fn).float()``.
    """
    return _e4m3_table()[np.asarray(q, dtype=np.uint8)]


NAN_TORCH = "torch"          # torch.clamp keeps a NaN: byte 0x7F | sign of the input
NAN_CLAMP_MIN = "clamp_min"  # Triton's tl.minimum(tl.maximum(x, -448), 448): -448, byte 0xFE


def quantize_e4m3(x: np.ndarray, scale: float = 1.0, nan: str = NAN_TORCH) -> np.ndarray:
    """q = e4m3fn(clamp(float32(x) / scale, -448, 448)).

    At scale 1.0 this is ``fp8_kv.quantize`` (fp8_kv.py:75-77) and the
    reference's FP8 append (reshape_and_cache.py:66-77); the division by a
    per-tensor fp32 scale is the build's extension.  A NaN quotient follows
    ``nan``: NAN_TORCH, torch.clamp's propagation (fp8_kv.quantize), stores
    0x7F with the input's sign; NAN_CLAMP_MIN, the append's Triton clamp,
    stores -448 (0xFE): tl.minimum / tl.maximum default to PropagateNan.NONE,
    i.e. LLVM minnum / maxnum, which return the non-NaN operand
    (triton/language/core.py:2506,2528 and semantic.py:380-381, Triton 3.6).
    """
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        y = (x / np.float32(scale)).astype(np.float32)
    nanq = np.isnan(y)
    y = np.where(nanq, np.float32(0.0), np.clip(y, -FP8_E4M3_MAX, FP8_E4M3_MAX)).astype(np.float32)
    q = e4m3fn_from_f32(y)
    if nan == NAN_CLAMP_MIN:
        q[nanq] = 0xFE
    elif nan == NAN_TORCH:
        q[nanq] = 0x7F | (np.signbit(x[nanq]).astype(np.uint8) << 7)
    else:
        raise ValueError(f"unknown NaN policy {nan}")
    return q


def dequantize_e4m3(q: np.ndarray, scale: float, out_dtype: str) -> np.ndarray:
    """y = round_out_dtype(float32(q) * scale) (build-defined gather dequant)."""
    with np.errstate(invalid="ignore", over="ignore"):
        y = (e4m3fn_to_f32(q) * np.float32(scale)).astype(np.float32)
    return from_f32(y, out_dtype)


# --------------------------------------------------------------------------- #
# append (MHA/GQA), reshape_and_cache.py:11-80
# --------------------------------------------------------------------------- #


def _slot_parts(slot_mapping, block_size, num_blocks):
    slots = np.asarray(slot_mapping, dtype=np.int64)
    tok = np.flatnonzero((slots >= 0) & (slots < num_blocks * block_size))  # :33-34
    s = slots[tok]
    return tok, s // block_size, s % block_size  # :36-37


def _write_rows(cache, tok, blk, off, rows, in_dtype, cache_dtype, scale):
    if cache_dtype == in_dtype:
        vals = rows[tok]
    elif cache_dtype == "fp8":
        vals = quantize_e4m3(to_f32(rows[tok], in_dtype), 1.0 if scale is None else scale, NAN_CLAMP_MIN)
    else:
        raise ValueError(f"cache dtype {cache_dtype} vs input {in_dtype}")
    cache[blk, off] = vals.reshape((len(tok),) + cache.shape[2:])


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, in_dtype="bf16", cache_dtype="bf16",
                      k_scale=None, v_scale=None):
    """In-place paged append; reshape_and_cache.py:11-80 (kernel), :83-135 (wrapper).

    key/value: [N, H, D] raw arrays.  key_cache/value_cache: [P, ps, H, D]
    arrays (views of a fused [P, 2, ps, H, D] tensor are fine).  For every
    token t with 0 <= slot < P*ps: cache[slot // ps, slot % ps] = q(x[t]).
    Other slots are untouched.
    """
    ps = key_cache.shape[1]
    tok, blk, off = _slot_parts(slot_mapping, ps, key_cache.shape[0])
    _write_rows(key_cache, tok, blk, off, np.asarray(key), in_dtype, cache_dtype, k_scale)
    _write_rows(value_cache, tok, blk, off, np.asarray(value), in_dtype, cache_dtype, v_scale)


def concat_and_cache_mla(kv_c, k_pe, kv_cache, slot_mapping, in_dtype="bf16", cache_dtype="bf16", scale=None):
    """MLA latent append; reshape_and_cache.py:138-188 (kernel), :191-229 (wrapper).

    kv_c: [N, Lk], k_pe: [N, Lv] (flat per token, reference :176-185);
    kv_cache: [P, ps, Lk + Lv].  cache[slot // ps, slot % ps] = [kv_c[t] | k_pe[t]].
    """
    ps = kv_cache.shape[1]
    kv_c = np.asarray(kv_c).reshape(kv_c.shape[0], -1)
    k_pe = np.asarray(k_pe).reshape(k_pe.shape[0], -1)
    tok, blk, off = _slot_parts(slot_mapping, ps, kv_cache.shape[0])
    row = np.concatenate([kv_c[tok], k_pe[tok]], axis=1)
    if cache_dtype == in_dtype:
        kv_cache[blk, off] = row.reshape((len(tok),) + kv_cache.shape[2:])
    elif cache_dtype == "fp8":
        q = quantize_e4m3(to_f32(row, in_dtype), 1.0 if scale is None else scale, NAN_CLAMP_MIN)
        kv_cache[blk, off] = q.reshape((len(tok),) + kv_cache.shape[2:])
    else:
        raise ValueError(f"cache dtype {cache_dtype} vs input {in_dtype}")


# --------------------------------------------------------------------------- #
# tile-scaled FP8 MLA entries (build-defined; the scheme the reference names
# when it rejects FP8 for MLA, pipeswift/utils/arguments.py:459-467)
# --------------------------------------------------------------------------- #

MLA_TILE = 128
MLA_MIN_TILE_SCALE = np.float32(2.0 ** -126)


def mla_tile_entry_bytes(nope_len, rope_len):
    """nope_len E4M3 bytes, one float32 scale per 128-element tile, rope_len bf16."""
    return nope_len + 4 * (nope_len // MLA_TILE) + 2 * rope_len


def quantize_mla_tiles(kv_c, k_pe):
    """kv_c [N, nope] and k_pe [N, rope] bf16 bits -> [N, entry] uint8 entries.

    Tile j of a row: amax_j = max |x| (NaN ignored), s_j = max(amax_j / 448,
    2^-126) in fp32, q = e4m3fn(clamp(x / s_j, -448, 448)), then the tile
    scales as float32 and the rope part as bf16 bit copies.  A NaN quotient
    (a NaN input, or +-inf / inf in a tile holding an infinity) stores 0x7F
    with the input's sign.
    """
    kv_c = np.asarray(kv_c, dtype=np.uint16)
    k_pe = np.asarray(k_pe, dtype=np.uint16)
    n, nope = kv_c.shape
    assert k_pe.ndim == 2 and k_pe.shape[0] == n
    tiles = nope // MLA_TILE
    x = bf16_to_f32(kv_c).reshape(n, tiles, MLA_TILE)
    a = np.abs(x)
    amax = np.where(np.isnan(a), np.float32(0), a).max(axis=2, initial=np.float32(0)).astype(np.float32)
    with np.errstate(over="ignore"):
        s = np.maximum((amax / np.float32(FP8_E4M3_MAX)).astype(np.float32), MLA_MIN_TILE_SCALE)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        y = (x / s[:, :, None]).astype(np.float32)
    y = np.where(np.isnan(y), np.copysign(np.float32(np.nan), x), np.clip(y, -FP8_E4M3_MAX, FP8_E4M3_MAX))
    y = y.astype(np.float32)
    out = np.empty((n, mla_tile_entry_bytes(nope, k_pe.shape[1])), dtype=np.uint8)
    out[:, :nope] = e4m3fn_from_f32(y).reshape(n, nope)
    out[:, nope: nope + 4 * tiles] = np.ascontiguousarray(s).view(np.uint8).reshape(n, 4 * tiles)
    out[:, nope + 4 * tiles:] = np.ascontiguousarray(k_pe).view(np.uint8).reshape(n, -1)
    return out


def dequantize_mla_tiles(entries, nope_len, out_dtype="bf16"):
    """[N, entry] uint8 -> [N, nope + rope] raw out_dtype bits:
    y = round(float32(q) * s_tile) for the nope part, the rope part exactly."""
    entries = np.ascontiguousarray(entries, dtype=np.uint8)
    n = entries.shape[0]
    tiles = nope_len // MLA_TILE
    s = np.ascontiguousarray(entries[:, nope_len: nope_len + 4 * tiles]).view(np.float32).reshape(n, tiles)
    with np.errstate(invalid="ignore", over="ignore"):
        y = (e4m3fn_to_f32(entries[:, :nope_len]).reshape(n, tiles, MLA_TILE) * s[:, :, None]).astype(np.float32)
    rope = np.ascontiguousarray(entries[:, nope_len + 4 * tiles:]).view(np.uint16).reshape(n, -1)
    nope_out = from_f32(y.reshape(n, nope_len), out_dtype)
    rope_out = rope if out_dtype == "bf16" else bf16_to_f32(rope).view(np.uint32)
    return np.concatenate([nope_out, rope_out.astype(nope_out.dtype)], axis=1)


def concat_and_cache_mla_tiles(kv_c, k_pe, cache, slot_mapping):
    """cache [P, ps, entry] uint8: the entry of every valid slot (as the GQA
    append skips negative and out-of-range slots) = quantize_mla_tiles(row)."""
    ps = cache.shape[1]
    tok, blk, off = _slot_parts(slot_mapping, ps, cache.shape[0])
    cache[blk, off] = quantize_mla_tiles(np.asarray(kv_c)[tok], np.asarray(k_pe)[tok])


def gather_mla_tiles(cache, block_table, cu_seq_lens, nope_len, seq_starts=None, out=None, out_dtype="bf16"):
    """gather_cache over the entries, then dequantize_mla_tiles; rows with no
    valid block are zeros, rows outside [cu[0], cu[-1]) of ``out`` untouched."""
    cu = np.asarray(cu_seq_lens, dtype=np.int64)
    rows = int(cu[-1]) if out is None else out.shape[0]
    entries = gather_cache(cache, block_table, cu, seq_starts, out=np.zeros((rows, cache.shape[2]), np.uint8),
                           cache_dtype="fp8")
    vals = dequantize_mla_tiles(entries, nope_len, out_dtype)
    if out is None:
        out = np.zeros_like(vals)
    written = np.zeros(rows, dtype=bool)
    written[int(cu[0]): min(int(cu[-1]), rows)] = True
    out[written] = vals[written]
    return out


# --------------------------------------------------------------------------- #
# gather (build-defined; vLLM gather_cache convention)
# --------------------------------------------------------------------------- #


def gather_cache(cache, block_table, cu_seq_lens, seq_starts=None, out=None, cache_dtype="bf16", out_dtype=None,
                 scale=None):
    """Contiguous rows from a paged cache.

    For sequence b and output token t in [cu[b], cu[b+1]):
    p = seq_starts[b] + t - cu[b] (seq_starts defaults to 0),
    out[t] = dq(cache[block_table[b, p // ps], p % ps]).
    A block id outside [0, P) or a page index beyond the table row gives a
    zero row.  The reference has no such op: its attention kernels read the
    cache through the same page_table (attention.py:189-211).
    """
    out_dtype = out_dtype or cache_dtype
    ps = cache.shape[1]
    P = cache.shape[0]
    cu = np.asarray(cu_seq_lens, dtype=np.int64)
    bt = np.asarray(block_table, dtype=np.int64)
    B = len(cu) - 1
    T = int(cu[-1]) if out is None else out.shape[0]
    row_shape = cache.shape[2:]
    if out is None:
        out = np.zeros((T,) + row_shape, dtype=RAW[out_dtype])
    for b in range(B):
        n = int(cu[b + 1] - cu[b])
        if n <= 0:
            continue
        start = 0 if seq_starts is None else int(seq_starts[b])
        t = np.arange(n, dtype=np.int64)
        p = start + t
        page = p // ps
        inb = page < bt.shape[1]
        blk = np.full(n, -1, dtype=np.int64)
        blk[inb] = bt[b, page[inb]]
        good = (blk >= 0) & (blk < P)
        rows = np.zeros((n,) + row_shape, dtype=RAW[cache_dtype])
        rows[good] = cache[blk[good], (p % ps)[good]]
        if out_dtype == cache_dtype:
            vals = rows
        else:
            vals = dequantize_e4m3(rows, 1.0 if scale is None else scale, out_dtype)
            vals[~good] = 0
        dst = np.arange(cu[b], cu[b + 1])
        keep = dst < T
        out[dst[keep]] = vals[keep]
    return out


# --------------------------------------------------------------------------- #
# copy_blocks (build-defined; vLLM copy_blocks convention, snapshot semantics)
# --------------------------------------------------------------------------- #


def validate_block_mapping(block_mapping, num_blocks):
    """Preconditions for snapshot semantics: ids in range, unique destinations,
    destinations disjoint from sources.  Raises AssertionError like the
    reference's host-side checks (copy_engine.py:373-385)."""
    m = np.asarray(block_mapping, dtype=np.int64).reshape(-1, 2)
    assert ((m >= 0) & (m < num_blocks)).all(), "block id out of range"
    assert len(np.unique(m[:, 1])) == len(m), "duplicate destination block"
    assert not np.isin(m[:, 1], m[:, 0]).any(), "a destination block is also a source"


def copy_blocks(stack, block_mapping):
    """stack: [L, P, ...]; for every layer and pair (s, d): stack[l, d] = stack[l, s].

    All reads happen before any write (snapshot), which is what an overlap-free
    mapping gives any execution order.
    """
    m = np.asarray(block_mapping, dtype=np.int64).reshape(-1, 2)
    if len(m) == 0:
        return
    stack[:, m[:, 1]] = stack[:, m[:, 0]].copy()


# --------------------------------------------------------------------------- #
# FP8 amax -> scale (build-defined; the reference fixes scale = 1.0)
# --------------------------------------------------------------------------- #


def amax_scale(x, dtype="bf16", qmax=FP8_E4M3_MAX):
    """(scale, amax): amax = max |x| ignoring NaN; scale = amax / qmax in fp32,
    or 1.0 when amax == 0."""
    f = np.abs(to_f32(np.asarray(x), dtype)).ravel()
    f = f[~np.isnan(f)]
    amax = np.float32(f.max()) if f.size else np.float32(0.0)
    scale = np.float32(amax / np.float32(qmax)) if amax > 0 else np.float32(1.0)
    return scale, amax


# --------------------------------------------------------------------------- #
# L2 offload transport helpers, copy_engine.py
# --------------------------------------------------------------------------- #


def page_bytes(shapes_itemsizes):
    """Bytes of one page across every layer of every cache tensor
    (copy_engine.py:121-125): sum over caches of L * prod(shape[2:]) * itemsize."""
    total = 0
    for shape, itemsize in shapes_itemsizes:
        total += int(np.prod(shape[2:], dtype=np.int64)) * itemsize * shape[0]
    return total


def coalesce(src_ids, dst_ids):
    """Runs of pages that advance together on both tiers (copy_engine.py:407-427).

    Sort by source (stable), split wherever src or dst does not step by one.
    Returns (src_start, dst_start, run_len) as uint64 arrays.
    """
    src_ids = np.asarray(src_ids, dtype=np.uint64)
    dst_ids = np.asarray(dst_ids, dtype=np.uint64)
    order = np.argsort(src_ids, kind="stable")
    src = src_ids[order]
    dst = dst_ids[order]
    breaks = (src[1:] != src[:-1] + 1) | (dst[1:] != dst[:-1] + 1)
    starts = np.flatnonzero(np.concatenate(([True], breaks)))
    lens = np.diff(np.append(starts, len(src))).astype(np.uint64)
    return src[starts], dst[starts], lens


def slot_mapping(page_table_row, offset, num_tokens, page_size, dcp_deg=1, dcp_rank=0, dcp_interleave_size=1):
    """Slots of positions [offset, num_tokens) of one sequence (metadata.py:272-295).

    dcp_deg == 1: slot = page_table[pos // ps] * ps + pos % ps.
    DCP: tokens interleave over ranks in runs of dcp_interleave_size; a rank
    owns pos when (pos // interleave) % dcp == rank and writes it at
    local_pos = pos % interleave + pos // (interleave * dcp) * interleave into
    physical pages of ps // dcp slots; foreign tokens get -1.
    """
    out = []
    if dcp_deg == 1:
        for pos in range(offset, num_tokens):
            out.append(page_table_row[pos // page_size] * page_size + pos % page_size)
        return out
    phys = page_size // dcp_deg
    stride = dcp_interleave_size * dcp_deg
    for pos in range(offset, num_tokens):
        if (pos // dcp_interleave_size) % dcp_deg == dcp_rank:
            local = pos % dcp_interleave_size + pos // stride * dcp_interleave_size
            out.append(page_table_row[pos // page_size] * phys + local % phys)
        else:
            out.append(-1)
    return out


def dcp_kv_len(prefix_len, dcp_deg, dcp_rank, dcp_interleave_size):
    """Tokens of a prefix a DCP rank holds (metadata.py:246-255)."""
    n = prefix_len // (dcp_interleave_size * dcp_deg) * dcp_interleave_size
    rem = prefix_len % (dcp_interleave_size * dcp_deg)
    if rem >= (dcp_rank + 1) * dcp_interleave_size:
        n += dcp_interleave_size
    elif rem >= dcp_rank * dcp_interleave_size:
        n += rem % dcp_interleave_size
    return n


def next_decode_step(page_tables, positions, lens_kv_prev, page_size, dcp_deg=1, dcp_rank=0, dcp_interleave_size=1):
    """Slots and lens_kv of the next draft decode step (metadata.py:351-414):
    one token per sequence at positions[i]; lens_kv + 1 where the rank owns
    it.  A position without a page raises IndexError, as the reference's
    page-table subscript does (:376)."""
    slots, lens = [], []
    for row, pos, prev in zip(page_tables, positions, lens_kv_prev):
        row[pos // page_size]  # IndexError, as kv_page_table[seq_id][pos // ps]
        s = slot_mapping(row, pos, pos + 1, page_size, dcp_deg, dcp_rank, dcp_interleave_size)[0]
        slots.append(s)
        lens.append(prev + 1 if s >= 0 else prev)
    return np.array(slots, np.int64), np.array(lens, np.int32)


def graph_refresh(static, step, cg_bsz, pad_q_len=1):
    """set_graph_kvcacheinfo (cudagraph.py:75-118) on numpy arrays, in place.

    static / step: dicts of page_table [rows, W], slot_mapping, lens_q,
    lens_kv, cu_seqlens_q.  Copies the step's metadata into the leading part of
    the static arrays; when bsz != cg_bsz pads lens_q with pad_q_len,
    slot_mapping with -1, lens_kv and page_table[bsz:, :W] with 0, and
    cu_seqlens_q[bsz + 1:] with cu[bsz] + k * pad_q_len (k = 1, 2, ...)."""
    bsz, w = step["lens_q"].shape[0], step["page_table"].shape[1]
    n = step["slot_mapping"].shape[0]
    static["page_table"][:bsz, :w] = step["page_table"]
    static["slot_mapping"][:n] = step["slot_mapping"]
    static["lens_q"][:bsz] = step["lens_q"]
    static["lens_kv"][:bsz] = step["lens_kv"]
    static["cu_seqlens_q"][: bsz + 1] = step["cu_seqlens_q"][: bsz + 1]
    if bsz != cg_bsz:
        assert bsz < cg_bsz
        static["lens_q"][bsz:] = pad_q_len
        static["slot_mapping"][n:] = -1
        static["lens_kv"][bsz:] = 0
        static["page_table"][bsz:, :w] = 0
        tail = static["cu_seqlens_q"].shape[0] - bsz
        static["cu_seqlens_q"][bsz + 1:] = static["cu_seqlens_q"][bsz] + np.arange(pad_q_len, tail * pad_q_len,
                                                                                    pad_q_len, dtype=np.int64)
    return static


# --------------------------------------------------------------------------- #
# paged decode attention over an FP8 cache
# --------------------------------------------------------------------------- #


def paged_decode_attention(q, q_dtype, k_cache, v_cache, block_table, seq_lens, softmax_scale, q_descale=None,
                           k_descale=None, v_descale=None, cu_seqlens_q=None, causal=False):
    """Decode attention over an FP8 E4M3FN paged cache, in float64 (the
    semantics the reference gets from vLLM's FA3 fork,
    pipeswift/llms/layers/attention.py:148-187: FP8 query, descales per
    (sequence, kv head), here any values instead of the fixed 1.0 of
    fp8_kv.py:94-103; ``max_seqlen_q`` = attention.py:175, ``causal`` =
    attention.py:181).

    q: raw bits [TQ, Hq, D] of ``q_dtype`` ("fp8" is used as is, others are
    quantized as e4m3(q / q_descale)); k_cache, v_cache: uint8 [P, ps, Hkv, D];
    block_table: int [B, W]; seq_lens: int [B]; descales: float [B, Hkv] or None.
    cu_seqlens_q: int [B + 1], sequence b's query tokens at rows
    [cu[b], cu[b+1]) of q, its last positions; None: one token per sequence
    (TQ = B).  With ``causal`` query token i of n sees keys
    [0, seq_len - n + 1 + i) (FA's bottom-right alignment), else all of them.
    Returns (out [TQ, Hq, D], lse [TQ, Hq]) as float64; a query token that
    sees no key, and a row no sequence owns, gives zeros and lse = -inf.  Table
    entries outside [0, P) read as zero rows.
    """
    q = np.asarray(q)
    TQ, Hq, D = q.shape
    P, ps, Hkv, _ = k_cache.shape
    G = Hq // Hkv
    if cu_seqlens_q is None:
        cu = np.arange(TQ + 1)
    else:
        cu = np.asarray(cu_seqlens_q, dtype=np.int64)
    B = len(cu) - 1
    out = np.zeros((TQ, Hq, D), dtype=np.float64)
    lse = np.full((TQ, Hq), -np.inf, dtype=np.float64)
    ones = np.ones((B, Hkv), dtype=np.float32)
    qd_all = ones if q_descale is None else np.asarray(q_descale, dtype=np.float32)
    kd_all = ones if k_descale is None else np.asarray(k_descale, dtype=np.float32)
    vd_all = ones if v_descale is None else np.asarray(v_descale, dtype=np.float32)
    for b in range(B):
        n = int(seq_lens[b])
        c0, nq = int(cu[b]), int(cu[b + 1] - cu[b])
        if n == 0 or nq <= 0:
            continue
        # keys each query token sees
        lim = np.array([min(n, max(0, n - nq + 1 + i)) if causal else n for i in range(nq)])
        j = np.arange(n)
        pages = np.asarray(block_table[b], dtype=np.int64)[j // ps]
        ok = (pages >= 0) & (pages < P)
        rows = j % ps
        for h in range(Hkv):
            qd, kd, vd = float(qd_all[b, h]), float(kd_all[b, h]), float(vd_all[b, h])
            K = np.zeros((n, D), dtype=np.float64)
            V = np.zeros((n, D), dtype=np.float64)
            K[ok] = e4m3fn_to_f32(k_cache[pages[ok], rows[ok], h]).astype(np.float64)
            V[ok] = e4m3fn_to_f32(v_cache[pages[ok], rows[ok], h]).astype(np.float64)
            for i in range(nq):
                L = int(lim[i])
                if L == 0:
                    continue
                qs = q[c0 + i, h * G:(h + 1) * G]
                if q_dtype == "fp8":
                    qq = e4m3fn_to_f32(qs).astype(np.float64)
                else:
                    qq = e4m3fn_to_f32(quantize_e4m3(to_f32(qs, q_dtype), qd)).astype(np.float64)
                s = (qq @ K[:L].T) * (float(np.float32(softmax_scale)) * qd * kd)
                m = s.max(axis=1, keepdims=True)
                p = np.exp(s - m)
                den = p.sum(axis=1, keepdims=True)
                out[c0 + i, h * G:(h + 1) * G] = (p @ V[:L]) / den * vd
                lse[c0 + i, h * G:(h + 1) * G] = (m + np.log(den))[:, 0]
    return out, lse
