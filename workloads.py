"""Seeded synthetic inputs for the benchmark configurations of the KV path.

Every tensor is generated on the CPU with ``torch.Generator().manual_seed`` so
the GPU kernels and the CPU checker see identical bytes; callers move them to
the device.  Layouts reproduce the reference's strided views: the fused GQA
cache [P, 2, ps, H, D] with K = [:, 0] and V = [:, 1] (llm.py:252-264), K and V
as column slices of one qkv projection row (transformer.py:547-551), MLA k_pe
as a column slice of the latent projection (transformer.py:1813-1821).

Config numbering follows the benchmark plan:
  1  bf16 GQA append, Llama-3-8B shape          (config1_append)
  2  FP8 E4M3 decode append, 128 sequences       (config2_fp8_decode)
  3  chunked-prefill append + block gather, Qwen3 (config3_chunked)
  4  MLA latent append, DeepSeek-V3 shape        (config4_mla)
  5a copy_blocks over a 61-layer stack           (config5a_copy_blocks)
  5b swap of 8192 blocks through the L2 mirror   (config5b_swap)
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

SEEDS = {"1": 1001, "2": 1002, "3": 1003, "4": 1004, "5a": 1005, "5b": 1006}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


_SENTINEL_TILE = 64 << 20


def sentinel(shape, dtype, seed) -> torch.Tensor:
    """Seeded random bytes viewed as ``dtype``: pre-fill for whole-buffer
    compares, so that a stray store of any byte value shows.  Buffers over
    64 MiB repeat one seeded 64 MiB tile, each repeat XORed with its index
    (a 2 GiB cache in about a second instead of a quarter of a minute)."""
    nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
    rng = np.random.default_rng(seed)
    tile = rng.integers(0, 256, min(nbytes, _SENTINEL_TILE), dtype=np.uint8)
    out = np.empty(nbytes, dtype=np.uint8)
    for i, start in enumerate(range(0, nbytes, len(tile) or 1)):
        n = min(len(tile), nbytes - start)
        np.bitwise_xor(tile[:n], np.uint8(i & 0xFF), out=out[start:start + n])
    return torch.from_numpy(out).view(dtype).view(shape)


@dataclass
class AppendCase:
    """One paged append: qkv-sliced K/V, a fused cache and its slot mapping."""

    qkv: torch.Tensor            # [N, q + 2*H*D] input rows; key/value are column slices
    q_size: int
    num_heads: int
    head_size: int
    cache: torch.Tensor          # [P, 2, ps, H, D] fused cache (sentinel-filled)
    slot_mapping: torch.Tensor   # int64 [N]
    extra: dict = field(default_factory=dict)

    def key(self, qkv=None):
        qkv = self.qkv if qkv is None else qkv
        kv = self.num_heads * self.head_size
        return qkv[:, self.q_size: self.q_size + kv].view(-1, self.num_heads, self.head_size)

    def value(self, qkv=None):
        qkv = self.qkv if qkv is None else qkv
        kv = self.num_heads * self.head_size
        return qkv[:, self.q_size + kv: self.q_size + 2 * kv].view(-1, self.num_heads, self.head_size)

    @property
    def num_valid(self) -> int:
        return int((self.slot_mapping >= 0).sum())


def config1_append(seed=SEEDS["1"], num_tokens=512, num_blocks=4096, block_size=16, heads=8, head_size=128,
                   q_size=4096, pad_frac=0.05, cache_dtype=torch.bfloat16) -> AppendCase:
    """bf16 GQA append (Llama-3-8B): N=512 tokens of [8, 128], cache
    [4096, 16, 8, 128], slots a seeded permutation of all slots with 5% -1."""
    g = _gen(seed)
    kv = heads * head_size
    qkv = torch.randn(num_tokens, q_size + 2 * kv, generator=g).to(torch.bfloat16)
    slots = torch.randperm(num_blocks * block_size, generator=g)[:num_tokens].to(torch.int64)
    pad = torch.randperm(num_tokens, generator=g)[: int(round(pad_frac * num_tokens))]
    slots[pad] = -1
    cache = sentinel((num_blocks, 2, block_size, heads, head_size), cache_dtype, seed + 1)
    return AppendCase(qkv, q_size, heads, head_size, cache, slots)


def config2_fp8_decode(seed=SEEDS["2"], batch=128, num_blocks=65536, block_size=16, heads=8, head_size=128,
                       q_size=4096, ctx_lo=128, ctx_hi=32768) -> AppendCase:
    """FP8 decode append: 128 sequences x 1 token, bf16 ~N(0, 2) with 1% x20
    outliers, into a [65536, 16, 8, 128] E4M3FN cache.  Context lengths are
    log-uniform in [128, 32768]; each sequence owns ceil(ctx/16) blocks drawn
    without replacement (block 0 is never handed out, block_manager.py:151-152)
    and its new token sits at position ctx-1."""
    g = _gen(seed)
    kv = heads * head_size
    qkv = (torch.randn(batch, q_size + 2 * kv, generator=g) * 2.0)
    mask = torch.rand(batch, q_size + 2 * kv, generator=g) < 0.01
    qkv = torch.where(mask, qkv * 20.0, qkv).to(torch.bfloat16)
    u = torch.rand(batch, generator=g, dtype=torch.float64)
    ctx = torch.exp(math.log(ctx_lo) + u * (math.log(ctx_hi) - math.log(ctx_lo))).floor().to(torch.int64)
    pages = (ctx + block_size - 1) // block_size
    assert int(pages.sum()) < num_blocks, "block pool too small for the drawn contexts"
    perm = torch.randperm(num_blocks - 1, generator=g) + 1
    tables, off = [], 0
    slots = torch.empty(batch, dtype=torch.int64)
    for b in range(batch):
        n = int(pages[b])
        table = perm[off: off + n]
        off += n
        tables.append(table)
        p = int(ctx[b]) - 1
        slots[b] = int(table[p // block_size]) * block_size + p % block_size
    cache = sentinel((num_blocks, 2, block_size, heads, head_size), torch.float8_e4m3fn, seed + 1)
    return AppendCase(qkv, q_size, heads, head_size, cache, slots, {"ctx": ctx, "tables": tables})


def prefill_append(seed=SEEDS["2"] + 100, num_tokens=32768, num_blocks=65536, block_size=16, heads=8,
                   head_size=128, q_size=4096, fp8=True) -> AppendCase:
    """A prefill-sized append in config 2's geometry (Llama-3-8B K/V, bf16
    ~N(0, 2) with 1% x20 outliers, qkv rows of 6144): num_tokens consecutive
    positions of fresh sequences, whole pages drawn without replacement from
    a [65536, 16, 8, 128] cache (FP8 E4M3FN, or bf16), in page order.  The
    size where the append is bound by HBM, not by its launch."""
    g = _gen(seed)
    kv = heads * head_size
    kvp = torch.randn(num_tokens, 2 * kv, generator=g) * 2.0
    mask = torch.rand(num_tokens, 2 * kv, generator=g) < 0.01
    qkv = torch.zeros(num_tokens, q_size + 2 * kv, dtype=torch.bfloat16)  # the query columns are not read
    qkv[:, q_size:] = torch.where(mask, kvp * 20.0, kvp).to(torch.bfloat16)
    pages = (num_tokens + block_size - 1) // block_size
    assert pages < num_blocks
    perm = torch.randperm(num_blocks - 1, generator=g)[:pages] + 1
    t = torch.arange(num_tokens)
    slots = (perm[t // block_size] * block_size + t % block_size).to(torch.int64)
    dt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    cache = sentinel((num_blocks, 2, block_size, heads, head_size), dt, seed + 1)
    return AppendCase(qkv, q_size, heads, head_size, cache, slots)


@dataclass
class ChunkedCase:
    append: AppendCase
    block_table: torch.Tensor   # int32 [B, W]
    cu_seq_lens: torch.Tensor   # int32 [B + 1] over full sequence lengths (prefix + chunk)
    prefix: torch.Tensor        # int64 [B]
    chunk: torch.Tensor         # int64 [B]


def config3_chunked(seed=SEEDS["3"], num_seqs=6, batched_tokens=4096, block_size=16, heads=4, head_size=128,
                    q_size=4096, max_prefix=60000, num_blocks=32768,
                    cache_dtype=torch.bfloat16) -> ChunkedCase:
    """Chunked prefill (Qwen3, 4 kv heads x 128): 4096 new tokens split over 6
    sequences, each with a page-aligned prefix of 0-60k tokens already cached;
    block tables are shuffled random blocks of a 32768-block cache."""
    g = _gen(seed)
    cuts = torch.sort(torch.randperm(batched_tokens - 1, generator=g)[: num_seqs - 1] + 1).values
    bounds = torch.cat([torch.tensor([0]), cuts, torch.tensor([batched_tokens])])
    chunk = (bounds[1:] - bounds[:-1]).to(torch.int64)
    prefix = (torch.randint(0, max_prefix // block_size + 1, (num_seqs,), generator=g) * block_size).to(torch.int64)
    total = prefix + chunk
    pages = (total + block_size - 1) // block_size
    assert int(pages.sum()) < num_blocks
    W = int(pages.max())
    perm = torch.randperm(num_blocks - 1, generator=g) + 1
    bt = torch.zeros(num_seqs, W, dtype=torch.int32)
    off = 0
    slots = []
    for b in range(num_seqs):
        n = int(pages[b])
        bt[b, :n] = perm[off: off + n].to(torch.int32)
        off += n
        pos = torch.arange(int(prefix[b]), int(total[b]))
        slots.append(bt[b, pos // block_size].to(torch.int64) * block_size + pos % block_size)
    slot_mapping = torch.cat(slots)
    kv = heads * head_size
    qkv = torch.randn(batched_tokens, q_size + 2 * kv, generator=g).to(torch.bfloat16)
    cache = sentinel((num_blocks, 2, block_size, heads, head_size), cache_dtype, seed + 1)
    cu = torch.zeros(num_seqs + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(total, 0).to(torch.int32)
    return ChunkedCase(AppendCase(qkv, q_size, heads, head_size, cache, slot_mapping), bt, cu, prefix, chunk)


@dataclass
class MLACase:
    latent: torch.Tensor        # [N, q_lora + Lk + Lv]; k_pe is a column slice
    kv_c: torch.Tensor          # [N, Lk] contiguous (normed)
    q_lora: int
    cache: torch.Tensor         # [P, ps, Lk + Lv]
    slot_mapping: torch.Tensor

    def k_pe(self, latent=None):
        latent = self.latent if latent is None else latent
        lk = self.kv_c.shape[1]
        return latent[:, self.q_lora + lk:]


def config4_mla(seed=SEEDS["4"], num_tokens=4096, num_blocks=20000, block_size=64, kv_lora=512, rope=64,
                q_lora=1536, cache_dtype=torch.bfloat16, decode=False) -> MLACase:
    """MLA latent append (DeepSeek-V3): kv_c [N, 512] and k_pe [N, 64] (a
    column slice of the [N, 1536+576] projection, row stride 2112) into a
    [20000, 64, 576] cache.  Prefill: tokens fill the pages of seeded random
    blocks in order.  Decode: 128 tokens at seeded random positions of seeded
    random blocks."""
    g = _gen(seed + (100 if decode else 0))
    latent = torch.randn(num_tokens, q_lora + kv_lora + rope, generator=g).to(torch.bfloat16)
    kv_c = torch.randn(num_tokens, kv_lora, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_blocks - 1, generator=g) + 1
    if decode:
        blocks = perm[:num_tokens]
        offs = torch.randint(0, block_size, (num_tokens,), generator=g)
        slots = blocks.to(torch.int64) * block_size + offs
    else:
        pos = torch.arange(num_tokens)
        slots = perm[pos // block_size].to(torch.int64) * block_size + pos % block_size
    cache = sentinel((num_blocks, block_size, kv_lora + rope), cache_dtype, seed + 1)
    return MLACase(latent, kv_c, q_lora, cache, slots.to(torch.int64))


def config4_mla_fp8_tiles(decode=False, num_tokens=None, seed=SEEDS["4"]) -> MLACase:
    """Config 4 with the tile-scaled FP8 latent entry: the same kv_c, k_pe view
    and slots, a [20000, 64, 656] uint8 cache of seeded bytes, and kv_c rows
    spread over 2^-8..2^8 in magnitude (with x20 outliers on 1% of elements)
    so that the per-tile scales differ."""
    n = num_tokens or (128 if decode else 4096)
    case = config4_mla(seed=seed, num_tokens=n, decode=decode)
    g = _gen(seed + 7)
    mag = torch.exp2(torch.empty(n, 4, 1).uniform_(-8, 8, generator=g)).expand(n, 4, 128).reshape(n, 512)
    out = torch.rand(n, 512, generator=g) < 0.01
    kv_c = (case.kv_c.float() * mag * torch.where(out, 20.0, 1.0)).to(torch.bfloat16)
    P, ps = case.cache.shape[0], case.cache.shape[1]
    cache = sentinel((P, ps, 656), torch.uint8, seed + 8)
    return MLACase(case.latent, kv_c, case.q_lora, cache, case.slot_mapping)


def config5a_pairs(seed=SEEDS["5a"], num_pairs=2048, num_blocks=8192) -> torch.Tensor:
    """2048 (src, dst) pairs, sources and destinations disjoint (one permutation)."""
    perm = torch.randperm(num_blocks, generator=_gen(seed))
    return torch.stack([perm[:num_pairs], perm[num_pairs: 2 * num_pairs]], 1).to(torch.int64).contiguous()


def config5b_pages(seed=SEEDS["5b"], num_pages=8192, gpu_pages=16384, l2_pages=8192):
    """GPU page ids (seeded random, so runs are short) and L2 page ids."""
    g = _gen(seed)
    gpu = torch.randperm(gpu_pages - 1, generator=g)[:num_pages] + 1
    l2 = torch.randperm(l2_pages, generator=g)[:num_pages]
    return gpu.numpy().astype(np.int64), l2.numpy().astype(np.int64)


# algorithmic bytes per launch (the roofline numerator) ---------------------- #


def append_bytes(num_valid, num_tokens, heads, head_size, in_size, cache_size) -> int:
    """K and V of each valid token read once and written once, plus the
    int64 slot of every token."""
    return num_valid * 2 * heads * head_size * (in_size + cache_size) + num_tokens * 8


def gather_bytes(total_tokens, row_elems, cache_size, out_size, num_pages, parts=2) -> int:
    return total_tokens * parts * row_elems * (cache_size + out_size) + num_pages * 4


def mla_bytes(num_tokens, row_elems, in_size, cache_size) -> int:
    return num_tokens * row_elems * (in_size + cache_size) + num_tokens * 8


def mla_fp8_tiles_bytes(num_tokens, nope=512, rope=64) -> int:
    """bf16 kv_c and k_pe read, one tile-scaled FP8 entry written, int64 slot."""
    return num_tokens * ((nope + rope) * 2 + nope + 4 * (nope // 128) + 2 * rope + 8)


def copy_blocks_bytes(num_pairs, num_layers, block_bytes) -> int:
    return num_pairs * num_layers * block_bytes * 2 + num_pairs * 16
