"""Benchmark of the MI355X paged KV-cache path (one GPU).

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline] [--eager]

A step is one launch of the hot-path kernel over one batch of synthetic input
(one decode step's K/V append for one layer, by default).  Exactly K launches
are timed after W untimed ones, each over a different rotation set of inputs
and slot mappings (the rotation keeps the working set far above the 256 MB
Infinity Cache); inputs are resident in HBM before timing.  HIP events on the
launch stream bracket the K launches (time_launches): up to 32 launches are
queued behind a spin kernel, so that they run back to back with host
submission outside the timed region; longer runs are one HIP graph of the K
launches, replayed as the reference replays its decode step from a CUDA graph
(llm.py:634-681).  --eager times plain launches instead (the PMC profiling
runs use it).

The default run reports config 2 (the FP8 decode append) as the headline and
every other benchmark configuration under `secondary`, each a bounded run of
its own timed the same way (its own step count), with its own roofline and
torch CPU baseline:
  fp8_decode_write   config 2 with the scales recomputed each step (amax + append)
  kv_scales          config 2's per-tensor K/V scales alone (amax kernels)
  bf16_append        config 1: 512 tokens of Llama-3-8B K/V (8x128), 4096 blocks
  chunked_append     config 3: 4096 tokens of Qwen3 K/V (4x128), 32768 blocks
  gather             config 3: the 6 sequences (prefix + chunk) to rows
  mla_prefill / mla_decode, mla_prefill_fp8 / mla_decode_fp8
                     config 4: kv_c 512 + k_pe 64, block 64, 20000 blocks, bf16
                     or per-tensor FP8
  copy_blocks        config 5a: 2048 pairs over 61 layers of [8192, 2, 16, 8, 128]
  decode_attention   one decode step of FP8 paged attention over config 2's cache
  decode_attention_q4  the same with 4 causal query tokens per sequence
                     (speculative decode: 16 MFMA rows per kv head)
  fp8_prefill_append   the fused FP8 append at prefill size: 32768 tokens in
                     config 2's geometry (--tokens to change; bf16_prefill_append
                     without the quantizer), where HBM rather than the launch
                     bounds it
  swap               config 5b: 8192 scattered blocks x 8 layers (4 GiB) D2H + H2D
  prefill_attention  a chunked-prefill step of FP8 paged attention (config 3
                     geometry: 4096 query tokens over prefixes of 14k-45k),
                     the prefill kernel; MFMA-bound, so its value is TFLOP/s
                     against the 2.5 PFLOP/s dense bf16 peak (--chunked: the
                     decode reader over 2-token chunks of the same step)
  metadata           host us of prepare_kv_info (configs 2 and 3) and of the
                     graph static-metadata refresh, against the reference's way

Output: plain-text progress lines, then ONE compact JSON result line, the
last line of the run (nothing is written to stderr).  The full per-workload
records go to the --detail file (by default bench_detail.json in the output
folder that the box's results are copied back from).  Each record
carries:
  value            algorithmic HBM GB/s (bytes the kernel must move / time)
  roofline         the same per launch against MI355X's 8 TB/s peak, the HBM
                   traffic measured with rocprofv3 PMC counters (committed
                   under profiles/), when present, and the fraction of the
                   best device copy measured on this box in the same run
                   (`achievable`, copy_blocks_kernel over 1 GiB)
  copy_floor       for workloads under 64 MB: device us of the HIP runtime's
                   contiguous copy of the same bytes at the same size, timed
                   the same way (vs_launch > 1: the kernel beats that copy)
  wall_us_per_call_eager  host wall time per eager Python call (no graph)
  cpu_baseline     the reference's CPU path, timed on this host: torch
                   index_put_ / index_select / amax (copy_blocks: a snapshot
                   index copy; attention: torch fp32 softmax(QK^T)V) on host
                   tensors of the same layout, on all the process's CPUs
                   (`cores`) and on one (`value_1thread`)
  cpu_oracle       the numpy oracle on one thread (headline only)

Other workloads (--workload NAME runs one alone): any name above, and
  mla_fp8_tiles_prefill / mla_fp8_tiles_decode   config 4 into 656-byte FP8
                     entries with one scale per 128-element tile
  attention_shapes   decode attention on several batch shapes, balanced vs split
  l2_cycle           BlockManager store -> evict -> restore of an 8192-page prompt
                     (the default run includes a 2048-page cycle)
  swap_sweep         host-link GB/s vs bytes per page, per transport
  hbm_copy           1 GiB device copy (achievable-bandwidth reference and the
                     PMC calibration run)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
import warnings

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFS = 2500.0  # MI355X dense bf16 MFMA
PUBLISHED_H2D_64K_GBPS = 47.9  # the reference's H2D at 64 KiB per descriptor, H100 (copy_engine.py:15-21)
SPIN_CYCLES = 2_000_000  # shader clocks of the pre-timing spin (~1 ms at 2.4 GHz)
STEADY_STEPS = 2048  # launches per graph for the steady per-launch figure of the us workloads
# Longest run timed by the queued method; longer runs replay one graph.  A
# graph replay costs about 15 us once, while a dispatch from the queue costs
# about 0.35 us (append) to 6 us (attention call) more than one replayed from a
# graph: the queued method is the more faithful one below about 40 launches.
QUEUED_MAX = 32
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def progress(msg):
    """A plain-text progress line on stdout.  Only the final result line of a
    run is JSON, and nothing goes to stderr, so the result line is the last
    line of the run's combined output."""
    print(f"[bench] {msg}", flush=True)


def _cpu_threads():
    """Host threads for the all-cores CPU baseline: the CPUs this process may
    run on, capped by OMP_NUM_THREADS where the box sets it."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# --------------------------------------------------------------------------- #
# workloads: each returns (launch(i), info dict)
# --------------------------------------------------------------------------- #


def _affine_block_maps(R, num_blocks, gen, device):
    """R bijections b -> (a*b + c) mod num_blocks (num_blocks a power of two, a odd)."""
    import torch

    a = torch.randint(0, num_blocks // 2, (R,), generator=gen) * 2 + 1
    c = torch.randint(0, num_blocks, (R,), generator=gen)
    return a.to(device), c.to(device)


def setup_append(args, device, fp8, rescale=False):
    """Config 1 (bf16) or config 2 (FP8 decode) append.  With ``rescale`` a
    step is the whole FP8 write of a caller that recomputes its per-tensor
    scales every step: ``reshape_and_cache_flash_amax``, the amax partials of
    K and V, then the fused append that finishes the scales itself (two
    launches; before it, amax partials, finalize and append took three); its
    bytes add the amax read of K and V."""
    import torch

    import workloads
    from pipeswift_amd import cache_ops
    from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash, reshape_and_cache_flash_amax

    case = workloads.config2_fp8_decode() if fp8 else workloads.config1_append()
    ps, P = case.cache.shape[2], case.cache.shape[0]
    N = case.slot_mapping.shape[0]
    R = args.rotate
    gen = torch.Generator().manual_seed(99)
    dgen = torch.Generator(device=device).manual_seed(99)
    qkv = torch.empty((R,) + tuple(case.qkv.shape), dtype=torch.bfloat16, device=device)
    qkv.normal_(0.0, 2.0 if fp8 else 1.0, generator=dgen)
    qkv[0].copy_(case.qkv.to(device))
    a, c = _affine_block_maps(R, P, gen, device)
    base = case.slot_mapping.to(device)
    valid = base >= 0
    blk = torch.where(valid, base // ps, torch.zeros_like(base))
    slots = ((a.view(R, 1) * blk.view(1, N) + c.view(R, 1)) % P) * ps + (base % ps).view(1, N)
    slots = torch.where(valid.view(1, N), slots, torch.full_like(slots, -1)).contiguous()
    slots[0].copy_(base)
    cache = case.cache.to(device)
    k_scale = v_scale = None
    scales = torch.ones(2, dtype=torch.float32, device=device)
    if fp8:
        cache_ops.warmup(device)
        cache_ops.compute_kv_scales(case.key(qkv[0]), case.value(qkv[0]), out=scales)
        k_scale, v_scale = scales[0:1], scales[1:2]
    kc, vc = cache[:, 0], cache[:, 1]

    if rescale:
        def launch(i):
            q = qkv[i]
            reshape_and_cache_flash_amax(case.key(q), case.value(q), kc, vc, slots[i], scales_out=scales)
    else:
        def launch(i):
            q = qkv[i]
            reshape_and_cache_flash(case.key(q), case.value(q), kc, vc, slots[i], k_scale, v_scale)

    nbytes = workloads.append_bytes(case.num_valid, N, case.num_heads, case.head_size, 2, 1 if fp8 else 2)
    amax_bytes = 2 * N * case.num_heads * case.head_size * 2
    name = "fp8_decode_write" if rescale else ("fp8_decode_append" if fp8 else "bf16_append")
    info = {
        "name": name,
        "kernel": ("amax_partial_kernel + paged_append_small_amax_kernel" if rescale
                   else "paged_append_small_kernel"),  # the launch for batches under 1024 tokens
        "bytes": nbytes + (amax_bytes if rescale else 0),
        "tokens": case.num_valid,
        "dtype": "fp8_e4m3fn" if fp8 else "bf16",
        "config": {
            "workload": ("fp8_decode_write: amax -> scale + fused FP8 append (config 2)" if rescale
                         else "fp8_decode_append (config 2)" if fp8 else "bf16_append (config 1)"),
            "tokens": N, "valid_tokens": case.num_valid, "kv_heads": case.num_heads, "head_dim": case.head_size,
            "block_size": ps, "num_blocks": P, "in_dtype": "bf16",
            "cache_dtype": "fp8_e4m3fn" if fp8 else "bf16", "qkv_row_stride": case.qkv.shape[1],
            "scale": ("per-tensor, recomputed from amax every step" if rescale
                      else "per-tensor from amax" if fp8 else None),
        },
        "cpu": lambda b: cpu_append(case, fp8, b),
        "cpu_torch": lambda b: torch_cpu_append(case, fp8, b, rescale=rescale),
        "cpu_torch_what": (("torch amax/448 of K and V, then " if rescale else "torch ")
                           + ("index_put_ of fp8_kv.quantize(x / scale) rows" if fp8 else "index_put_ of the K/V rows")
                           + " into a host cache of the same layout"),
    }
    if rescale:
        info["config"]["amax_read_bytes"] = amax_bytes
    return launch, info


def setup_prefill_append(args, device, tokens=32768, fp8=True):
    """The fused append at prefill size (workloads.prefill_append): `tokens`
    new tokens of Llama-3-8B K/V into config 2's [65536, 16, 8, 128] cache,
    FP8 with per-tensor scales (or bf16).  Inputs rotate over enough sets that
    inputs and cache pages span >= 2 GiB, so neither L2 nor MALL holds them."""
    import math

    import torch

    import workloads
    from pipeswift_amd import cache_ops
    from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash

    q_size = 4096 if args.q_size < 0 else args.q_size
    bs = args.block_size  # 16 (config 2); larger pages as a sensitivity run over the same 2 GiB of slots
    case = workloads.prefill_append(num_tokens=tokens, fp8=fp8, q_size=q_size, block_size=bs,
                                    num_blocks=65536 * 16 // bs)
    ps, P = case.cache.shape[2], case.cache.shape[0]
    N = tokens
    row_bytes = case.qkv.shape[1] * 2
    R = max(2, min(args.rotate, math.ceil(2.5e9 / (N * row_bytes))))
    gen = torch.Generator().manual_seed(98)
    dgen = torch.Generator(device=device).manual_seed(98)
    qkv = torch.empty((R,) + tuple(case.qkv.shape), dtype=torch.bfloat16, device=device)
    qkv.normal_(0.0, 2.0, generator=dgen)
    qkv[0].copy_(case.qkv.to(device))
    a, c = _affine_block_maps(R, P, gen, device)
    base = case.slot_mapping.to(device)
    if args.slots == "contiguous":
        # every rotation set writes one run of consecutive slots (pages in
        # order): the same kernel without the page scatter
        start = (torch.arange(R, device=device) * N) % (P * ps - N + 1)
        slots = start.view(R, 1) + torch.arange(N, device=device).view(1, N)
    else:
        slots = ((a.view(R, 1) * (base // ps).view(1, N) + c.view(R, 1)) % P) * ps + (base % ps).view(1, N)
        slots[0].copy_(base)
    cache = case.cache.to(device)
    k_scale = v_scale = None
    if fp8:
        scales = torch.ones(2, dtype=torch.float32, device=device)
        cache_ops.warmup(device)
        cache_ops.compute_kv_scales(case.key(qkv[0]), case.value(qkv[0]), out=scales)
        k_scale, v_scale = scales[0:1], scales[1:2]
    kc, vc = cache[:, 0], cache[:, 1]

    def launch(i):
        q = qkv[i]
        reshape_and_cache_flash(case.key(q), case.value(q), kc, vc, slots[i], k_scale, v_scale)

    name = f"{'fp8' if fp8 else 'bf16'}_prefill_append" + ("" if tokens == 32768 else f"_{tokens}")
    info = {
        "name": name,
        "kernel": "paged_scatter_kernel" if N >= 1024 else "paged_append_small_kernel",
        "bytes": workloads.append_bytes(N, N, case.num_heads, case.head_size, 2, 1 if fp8 else 2),
        "tokens": N,
        "dtype": "fp8_e4m3fn" if fp8 else "bf16",
        "rotate": R,
        "config": {
            "workload": f"fused {'FP8' if fp8 else 'bf16'} append of {N} prefill tokens (config 2's cache geometry)",
            "tokens": N, "kv_heads": case.num_heads, "head_dim": case.head_size, "block_size": ps,
            "num_blocks": P, "in_dtype": "bf16", "cache_dtype": "fp8_e4m3fn" if fp8 else "bf16",
            "qkv_row_stride": case.qkv.shape[1], "scale": "per-tensor from amax" if fp8 else None,
        },
        "cpu": lambda b: cpu_append(case, fp8, b),
        "cpu_torch": lambda b: torch_cpu_append(case, fp8, b),
        "cpu_torch_what": ("torch index_put_ of fp8_kv.quantize(x / scale) rows" if fp8
                           else "torch index_put_ of the K/V rows") + " into a host cache of the same layout",
    }
    if q_size != 4096:
        info["name"] += f"_q{q_size}"
    if bs != 16:
        info["name"] += f"_bs{bs}"
    if args.slots == "contiguous":
        info["name"] += "_contiguous"
        info["config"]["slots"] = "one run of consecutive slots per rotation set"
    return launch, info


def setup_decode_attention(args, device, q_len=1):
    """One decode step of paged attention over config 2's FP8 cache: 128
    sequences with log-uniform 128-32768 token contexts in the
    [65536, 16, 8, 128] E4M3FN cache, 32 query heads (4 per kv head), per-tensor
    K/V descales.  q_len > 1: that many query tokens per sequence (speculative
    decode), causal.  Algorithmic bytes: every context token's K and V rows of
    every kv head, the page ids, the bf16 queries and the bf16 outputs."""
    import torch

    import workloads
    from pipeswift_amd import attention

    case = workloads.config2_fp8_decode()
    ctx, tables = case.extra["ctx"], case.extra["tables"]
    B, H, D, Hq, ps = 128, 8, 128, 32, 16
    cache = case.cache.to(device)
    dgen = torch.Generator(device=device).manual_seed(77)
    for p0 in range(0, cache.shape[0], 4096):  # random FP8 contents, 4096 pages at a time
        blk = cache[p0: p0 + 4096]
        blk.copy_((torch.randn(blk.shape, device=device, generator=dgen) * 2.0).to(torch.float8_e4m3fn))
    W = max(len(t) for t in tables)
    bt = torch.zeros(B, W, dtype=torch.int32)
    for b in range(B):
        bt[b, : len(tables[b])] = tables[b].to(torch.int32)
    bt = bt.to(device)
    lens = ctx.to(torch.int32).to(device)
    R = min(args.rotate, 64)
    q = (torch.randn(R, B * q_len, Hq, D, device=device, generator=dgen) * 2.0).to(torch.bfloat16)
    scales = torch.tensor([0.01, 0.02], dtype=torch.float32, device=device)
    out = torch.empty(B * q_len, Hq, D, dtype=torch.bfloat16, device=device)
    ws = torch.empty(attention.workspace_floats(B, Hq, H, W * ps, args.num_splits, q_len), dtype=torch.float32,
                     device=device)
    kc, vc = cache[:, 0], cache[:, 1]

    def launch(i):
        attention.paged_decode_attention(q[i], kc, vc, bt, lens, D ** -0.5, None, scales[0:1], scales[1:2], out=out,
                                         workspace=ws, num_splits=args.num_splits, q_len=q_len, causal=True)

    total = int(ctx.sum())
    pages = int(sum(len(t) for t in tables))
    nbytes = total * H * D * 2 + pages * 4 + 2 * B * q_len * Hq * D * 2
    config = {"workload": "FP8 paged decode attention (config 2 cache)", "sequences": B, "context_tokens": total,
              "kv_heads": H, "q_heads": Hq, "head_dim": D, "block_size": ps, "num_blocks": cache.shape[0],
              "num_splits": args.num_splits or "auto", "descales": "per-tensor K/V"}
    if q_len > 1:
        config["workload"] = f"FP8 paged attention, {q_len} causal query tokens per sequence (config 2 cache)"
        config["query_tokens_per_sequence"] = q_len
    info = {
        "name": "decode_attention" if q_len == 1 else f"decode_attention_q{q_len}",
        # the head-parallel balanced schedule from 2 sequences up, the split schedule for an explicit count
        "kernel": "decode_partial_heads_kernel" if args.num_splits == 0 else "decode_partial_ring_kernel",
        "bytes": nbytes, "tokens": B,
        "dtype": "fp8_e4m3fn",
        "rotate": R,
        "config": config,
        "cpu": lambda b: cpu_decode_attention(kc, vc, bt, ctx, q[0], scales, total * H * D * 2, b, q_len),
        "cpu_torch": lambda b: torch_cpu_decode_attention(kc, vc, bt, ctx, q[0], scales, nbytes, b, q_len),
        "cpu_torch_what": "torch fp32 attention (dequantized K/V pages, softmax(QK^T)V) over the first 16 "
                          "sequences, scaled to the whole batch's bytes",
    }
    return launch, info


def setup_prefill_attention(args, device):
    """A chunked-prefill step of attention over an FP8 paged cache, in config
    3's geometry: 4096 new query tokens over 6 sequences with page-aligned
    prefixes of 14k-45k cached tokens, 32 query heads over 4 kv heads, random
    FP8 pages, causal, per-tensor descales, through ``flash_attn_varlen_func``
    as the reference's ``_fp8_paged_attn`` calls it for prefill (the prefill
    kernel).  MFMA-bound: algorithmic FLOPs are 4 * 128 per visible (query
    head, key) pair (Q K^T and P V, 2 * 128 each), counted once, as the
    kernel runs them (P V once, on fp16 P).  Algorithmic
    bytes: every sequence's K and V rows once, the page ids, the bf16 queries
    and outputs.  ``--chunked`` times the decode reader over 2-token chunks of
    the same step instead."""
    import torch

    import workloads
    from pipeswift_amd import attention

    cc = workloads.config3_chunked()
    H, D, Hq, ps = 4, 128, 32, 16
    P = cc.append.cache.shape[0]
    dgen = torch.Generator(device=device).manual_seed(76)
    cache = (torch.randn((P, 2, ps, H, D), device=device, generator=dgen) * 2.0).to(torch.float8_e4m3fn)
    kc, vc = cache[:, 0], cache[:, 1]
    bt = cc.block_table.to(device)
    chunk = cc.chunk
    N = int(chunk.sum())
    cu = torch.zeros(len(chunk) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(chunk, 0).to(torch.int32)
    cu = cu.to(device)
    lens = (cc.prefix + cc.chunk).to(torch.int32).to(device)
    R = min(args.rotate, 4)
    q = (torch.randn(R, N, Hq, D, device=device, generator=dgen) * 2.0).to(torch.bfloat16)
    scales = torch.tensor([0.01, 0.02], dtype=torch.float32, device=device)
    out = torch.empty(N, Hq, D, dtype=torch.bfloat16, device=device)
    maxq = int(chunk.max())

    fn = attention.chunked_prefill_attention if getattr(args, "chunked", False) else attention.flash_attn_varlen_func
    ws = torch.empty(attention.prefill_workspace_words(len(chunk)), dtype=torch.int32, device=device)

    def launch(i):
        if fn is attention.flash_attn_varlen_func:
            attention.paged_prefill_attention(q[i], kc, vc, bt, lens, cu, maxq, D ** -0.5, None, scales[0:1],
                                              scales[1:2], out=out, causal=True, workspace=ws)
        else:
            fn(q[i], kc, vc, maxq, cu, lens, bt, softmax_scale=D ** -0.5, causal=True, k_descale=scales[0:1],
               v_descale=scales[1:2], out=out)

    total = int(lens.sum())
    pages = int(((cc.prefix + cc.chunk + ps - 1) // ps).sum())
    nbytes = total * H * D * 2 + pages * 4 + 2 * N * Hq * D * 2
    p, c = cc.prefix.double(), cc.chunk.double()
    pairs = float((c * p + c * (c + 1) / 2).sum()) * Hq  # visible (query head, key) pairs, causal
    kernel = ("decode_partial_ring_kernel + decode_combine_kernel" if fn is not attention.flash_attn_varlen_func
              else "prefill_attention_kernel")
    flops = 4.0 * D * pairs

    def cpu_torch(budget):
        # the last 32 query tokens of sequence 0, every head, scaled by FLOPs
        L0, e0 = int(lens[0]), int(cu[1])
        step, _, _ = torch_cpu_decode_attention_step(kc, vc, bt[:1], lens[:1].cpu(), q[0][e0 - 32:e0], scales, 32, 1)
        n, el = _timed(step, budget)
        return n * 4.0 * D * Hq * sum(L0 - 31 + r for r in range(32)) / flops, el
    return launch, {
        "name": "prefill_attention", "kernel": kernel, "flops": flops, "cpu_torch": cpu_torch,
        "cpu_torch_what": "torch fp32 causal attention on host tensors (the last 32 query tokens of sequence 0, "
                          "all heads; scaled by FLOPs)",
        "bytes": nbytes, "tokens": N, "dtype": "fp8_e4m3fn", "rotate": R,
        "config": {"workload": "chunked-prefill attention over an FP8 paged cache (config 3 geometry)",
                   "query_tokens": N, "context_tokens": total, "q_heads": Hq, "kv_heads": H, "head_dim": D,
                   "block_size": ps, "path": "chunked decode reader" if kernel.startswith("decode") else
                   "prefill kernel"},
    }


def setup_kv_scales(args, device):
    """Per-tensor FP8 scales of config 2's K and V (amax / 448), one launch."""
    import torch

    import workloads
    from pipeswift_amd import cache_ops

    case = workloads.config2_fp8_decode()
    R = args.rotate
    dgen = torch.Generator(device=device).manual_seed(93)
    qkv = torch.empty((R,) + tuple(case.qkv.shape), dtype=torch.bfloat16, device=device)
    qkv.normal_(0.0, 2.0, generator=dgen)
    out = torch.empty(2, dtype=torch.float32, device=device)
    cache_ops.warmup(device)

    def launch(i):
        q = qkv[i]
        cache_ops.compute_kv_scales(case.key(q), case.value(q), out=out)

    nbytes = 2 * case.qkv.shape[0] * case.num_heads * case.head_size * 2
    return launch, {
        "name": "kv_scales", "kernel": "amax_partial_kernel + amax_finalize_kernel", "bytes": nbytes, "tokens": case.qkv.shape[0],
        "dtype": "bf16",
        "config": {"workload": "FP8 per-tensor scale from amax, config 2 K and V", "tokens": case.qkv.shape[0]},
        "cpu": None,
        "cpu_torch": lambda b: torch_cpu_kv_scales(case, b),
        "cpu_torch_what": "torch amax(|x|) / 448 of K and of V on the host",
    }


def setup_chunked(args, device, gather):
    import torch

    import workloads
    from pipeswift_amd import cache_ops
    from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash

    # --block-size: the sensitivity run at a larger page (the same token
    # capacity: num_blocks scaled down)
    ps_arg = args.block_size
    cc = workloads.config3_chunked(block_size=ps_arg, num_blocks=32768 * 16 // ps_arg)
    a = cc.append
    P, ps = a.cache.shape[0], a.cache.shape[2]
    cache = a.cache.to(device)
    R = args.rotate if not gather else max(1, min(args.rotate, 8))
    gen = torch.Generator().manual_seed(98)
    am, cm = _affine_block_maps(R, P, gen, device)
    if not gather:
        N = a.slot_mapping.shape[0]
        dgen = torch.Generator(device=device).manual_seed(98)
        qkv = torch.empty((R,) + tuple(a.qkv.shape), dtype=torch.bfloat16, device=device)
        qkv.normal_(generator=dgen)
        base = a.slot_mapping.to(device)
        slots = ((am.view(R, 1) * (base // ps).view(1, N) + cm.view(R, 1)) % P) * ps + (base % ps).view(1, N)
        kc, vc = cache[:, 0], cache[:, 1]

        def launch(i):
            q = qkv[i]
            reshape_and_cache_flash(a.key(q), a.value(q), kc, vc, slots[i])

        nbytes = workloads.append_bytes(N, N, a.num_heads, a.head_size, 2, 2)
        return launch, {
            "name": "chunked_append", "kernel": "paged_scatter_kernel", "bytes": nbytes, "tokens": N,
            "dtype": "bf16",
            "config": {"workload": "chunked_append (config 3)" + ("" if ps == 16 else f", block size {ps}"), "tokens": N, "kv_heads": a.num_heads,
                       "head_dim": a.head_size, "block_size": ps, "num_blocks": P, "sequences": len(cc.chunk)},
            "cpu": lambda b: cpu_append(a, False, b),
            "cpu_torch": lambda b: torch_cpu_append(a, False, b),
            "cpu_torch_what": "torch index_put_ of the K/V rows into a host cache of the same layout",
        }
    T = int(cc.cu_seq_lens[-1])
    bt = cc.block_table.to(device)
    bts = ((am.view(R, 1, 1) * bt.long().view(1, *bt.shape) + cm.view(R, 1, 1)) % P).to(torch.int32).contiguous()
    cu = cc.cu_seq_lens.to(device)
    out_k = torch.empty(T, a.num_heads, a.head_size, dtype=torch.bfloat16, device=device)
    out_v = torch.empty_like(out_k)
    kc, vc = cache[:, 0], cache[:, 1]

    def launch(i):
        cache_ops.gather_cache(kc, out_k, bts[i], cu, src_cache_v=vc, dst_v=out_v)

    pages = int(((cc.prefix + cc.chunk + ps - 1) // ps).sum())
    nbytes = workloads.gather_bytes(T, a.num_heads * a.head_size, 2, 2, pages)
    return launch, {
        "name": "gather", "kernel": "paged_gather_kernel", "bytes": nbytes, "tokens": T, "dtype": "bf16",
        "rotate": R,
        "config": {"workload": "block gather (config 3)" + ("" if ps == 16 else f", block size {ps}"), "tokens": T, "sequences": len(cc.chunk),
                   "kv_heads": a.num_heads, "head_dim": a.head_size, "block_size": ps, "num_blocks": P,
                   "pages": pages},
        "cpu": lambda b: cpu_gather(cc, b),
        "cpu_torch": lambda b: torch_cpu_gather(cc, b),
        "cpu_torch_what": "torch index_select of each sequence's K and V pages, reshaped to rows",
    }


def setup_mla(args, device, decode, fp8=False):
    """Config 4's MLA latent append, prefill (4096 tokens) or decode (128),
    into the bf16 cache or, with ``fp8``, an E4M3FN cache with one per-tensor
    scale (amax of kv_c and k_pe over 448, computed once at set-up)."""
    import torch

    import workloads
    from pipeswift_amd import cache_ops
    from pipeswift_amd.reshape_and_cache import reshape_and_cache_flash_diffkv

    n = args.tokens or (128 if decode else 4096)
    case = workloads.config4_mla(num_tokens=n, decode=decode)
    P, ps = case.cache.shape[0], case.cache.shape[1]
    R = args.rotate
    dgen = torch.Generator(device=device).manual_seed(97)
    latent = torch.empty((R,) + tuple(case.latent.shape), dtype=torch.bfloat16, device=device)
    latent.normal_(generator=dgen)
    kv_c = torch.empty((R,) + tuple(case.kv_c.shape), dtype=torch.bfloat16, device=device)
    kv_c.normal_(generator=dgen)
    latent[0].copy_(case.latent.to(device))
    kv_c[0].copy_(case.kv_c.to(device))
    slots = torch.stack([torch.randperm(P * ps, generator=torch.Generator().manual_seed(97 + r))[:n]
                         for r in range(min(R, 64))]).to(torch.int64).to(device)
    slots[0].copy_(case.slot_mapping.to(device))
    scale = None
    if fp8:
        cache = torch.zeros(tuple(case.cache.shape), dtype=torch.uint8, device=device).view(torch.float8_e4m3fn)
        cache_ops.warmup(device)
        sc = torch.empty(2, dtype=torch.float32, device=device)
        cache_ops.compute_kv_scales(kv_c[0], out=sc[0:1])
        cache_ops.compute_kv_scales(case.k_pe(latent[0]), out=sc[1:2])
        scale = sc.max().reshape(1).contiguous()  # one scale for the whole row: max of the two amax / 448
    else:
        cache = case.cache.to(device)
    cache = cache.unsqueeze(2)

    def launch(i):
        reshape_and_cache_flash_diffkv(kv_c[i].unsqueeze(1), case.k_pe(latent[i]).unsqueeze(1), cache,
                                       slots[i % slots.shape[0]], scale)

    nbytes = workloads.mla_bytes(n, 576, 2, 1 if fp8 else 2)
    kind = "decode" if decode else "prefill"
    name = f"mla_{kind}" + ("_fp8" if fp8 else "") + ("" if n == (128 if decode else 4096) else f"_{n}")
    host_scale = None if scale is None else float(scale.cpu())
    return launch, {
        "rotate": R,
        "name": name,
        "kernel": ("paged_append_small_kernel" if n < 1024 else
                   "packed_row_scatter_kernel" if fp8 else "paged_scatter_kernel"), "bytes": nbytes,
        "tokens": n, "dtype": "fp8_e4m3fn" if fp8 else "bf16",
        "config": {"workload": f"MLA latent append, {kind}" + (", per-tensor FP8" if fp8 else "") + " (config 4)",
                   "tokens": n, "row": 576, "block_size": ps, "num_blocks": P,
                   "cache_dtype": "fp8_e4m3fn" if fp8 else "bf16"},
        "cpu": None,
        "cpu_torch": lambda b: torch_cpu_mla(case, host_scale, b),
        "cpu_torch_what": ("torch index_put_ of the [kv_c | k_pe] rows" + (" after fp8_kv.quantize(x / scale)"
                           if fp8 else "") + " into a host [P, 64, 576] cache"),
    }


def setup_mla_fp8_tiles(args, device, decode):
    """Config 4 into the tile-scaled FP8 latent entry (656 bytes per token)."""
    import torch

    import workloads
    from pipeswift_amd import mla_fp8

    case = workloads.config4_mla_fp8_tiles(decode=decode)
    n = case.slot_mapping.shape[0]
    P, ps = case.cache.shape[0], case.cache.shape[1]
    R = args.rotate
    dgen = torch.Generator(device=device).manual_seed(98)
    latent = torch.empty((R,) + tuple(case.latent.shape), dtype=torch.bfloat16, device=device)
    latent.normal_(generator=dgen)
    kv_c = torch.empty((R,) + tuple(case.kv_c.shape), dtype=torch.bfloat16, device=device)
    kv_c.normal_(generator=dgen)
    slots = torch.stack([torch.randperm(P * ps, generator=torch.Generator().manual_seed(98 + r))[:n]
                         for r in range(min(R, 64))]).to(torch.int64).to(device)
    slots[0].copy_(case.slot_mapping.to(device))
    cache = case.cache.to(device)

    def launch(i):
        mla_fp8.concat_and_cache_mla_fp8_tiles(kv_c[i], case.k_pe(latent[i]), cache, slots[i % slots.shape[0]])

    name = "mla_fp8_tiles_decode" if decode else "mla_fp8_tiles_prefill"
    return launch, {
        "rotate": R,
        "name": name, "kernel": "tile_fp8_append_kernel", "bytes": workloads.mla_fp8_tiles_bytes(n),
        "tokens": n, "dtype": "bf16->fp8_e4m3fn",
        "config": {"workload": f"MLA latent append into tile-scaled FP8 entries, {'decode' if decode else 'prefill'}"
                               " (config 4)", "tokens": n, "entry_bytes": 656, "block_size": ps, "num_blocks": P},
        "cpu": lambda b: cpu_mla_fp8_tiles(case, b),
    }


def setup_copy_blocks(args, device):
    import torch

    import workloads
    from pipeswift_amd import cache_ops

    L, P = 61, 8192
    stack = torch.empty((L, P, 2, 16, 8, 128), dtype=torch.bfloat16, device=device)
    stack.view(torch.int16).random_(generator=torch.Generator(device=device).manual_seed(96))
    pairs = [workloads.config5a_pairs(seed=1005 + r).to(device) for r in range(4)]

    def launch(i):
        cache_ops.copy_blocks(stack, pairs[i % len(pairs)], validate=False)

    nbytes = workloads.copy_blocks_bytes(2048, L, 2 * 16 * 8 * 128 * 2)
    return launch, {
        "rotate": len(pairs),
        "name": "copy_blocks", "kernel": "copy_blocks_kernel", "bytes": nbytes, "tokens": 2048 * 16,
        "dtype": "bf16",
        "config": {"workload": "copy_blocks (config 5a)", "pairs": 2048, "layers": L, "num_blocks": P,
                   "block_bytes": 65536},
        "cpu": lambda b: cpu_copy_blocks(nbytes, b),
        "cpu_torch": lambda b: torch_cpu_copy_blocks(nbytes, b),
        "cpu_torch_what": "torch snapshot index copy stack[:, dst] = stack[:, src].clone() over 128 pairs of a "
                          "61-layer 256-block host stack, scaled to config 5a's bytes",
    }


def measure_device_copy(device, reps=10):
    """GB/s (read + write) of the best device copy on this box: copy_blocks_kernel
    over 16384 contiguous 64 KiB blocks, 1 GiB each way.  The achievable
    reference of the roofline next to the 8 TB/s spec."""
    import torch

    from pipeswift_amd import cache_ops

    stack = torch.empty((1, 2 * 16384, 65536), dtype=torch.uint8, device=device)
    pairs = torch.stack([torch.arange(16384), torch.arange(16384) + 16384], 1).to(torch.int64).to(device)
    for _ in range(3):
        cache_ops.copy_blocks(stack, pairs, validate=False)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        cache_ops.copy_blocks(stack, pairs, validate=False)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * (1 << 30) / (e0.elapsed_time(e1) / 1e3 / reps) / 1e9
    del stack
    torch.cuda.empty_cache()
    return gbs


def measure_copy_floor(device, nbytes, steps=256):
    """Device microseconds of the HIP runtime's own contiguous copy (torch
    ``copy_``) moving the same bytes as one launch (nbytes / 2 each way), over
    rotated buffer pairs (a working set of at least 1 GiB, above the Infinity
    Cache), `steps` copies timed as the workload's launches are: the floor of
    a plain copy at this size, for the microsecond workloads."""
    import torch

    each = max(16, (nbytes // 2) // 16 * 16)
    n = int(min(512, max(16, math.ceil((1 << 30) / (2 * each)))))
    src = torch.zeros(n, each, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    t = time_launches(lambda i: dst[i].copy_(src[i]), n, steps, 16, device, eager_calls=1)
    del src, dst
    torch.cuda.empty_cache()
    return t["ms"] * 1e3 / t["launches"]


def run_hbm_copy(args, device):
    """Achievable-bandwidth reference: a 1 GiB device-to-device copy, once with
    torch (the runtime's copy kernel) and once with copy_blocks_kernel over
    16384 contiguous 64 KiB blocks; also the PMC calibration workload (each
    dispatch must read and write exactly 1 GiB)."""
    import torch

    from pipeswift_amd import cache_ops

    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device=device)
    a.random_(generator=torch.Generator(device=device).manual_seed(94))
    b = torch.empty_like(a)
    out = {}
    stack = torch.empty((1, 2 * 16384, 65536), dtype=torch.uint8, device=device)
    pairs = torch.stack([torch.arange(16384), torch.arange(16384) + 16384], 1).to(torch.int64).to(device)
    for name, fn in (("torch_copy", lambda: b.copy_(a)),
                     ("copy_blocks_kernel", lambda: cache_ops.copy_blocks(stack, pairs, validate=False))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = 2 * n / (e0.elapsed_time(e1) / 1e3 / reps) / 1e9
    line = {"metric": "device copy GB/s (read + write), 1 GiB", "value": round(max(out.values()), 2), "unit": "GB/s",
            "n_gpus": 1, "steps": 20, "warmup": 3, "higher_is_better": True, "vs_baseline": None, "dtype": "bytes",
            "data": "synthetic", "config": {"workload": "hbm_copy (roofline reference)", "results": out},
            "roofline": {"bound": "hbm", "achieved": round(max(out.values()), 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(max(out.values()) / PEAK_HBM_GBS, 4), "traffic": None}}
    print(json.dumps(line), flush=True)


def measure_swap(device, transports=("blit",), reps=3):
    """D2H store then H2D load of 8192 scattered blocks x 8 layers (4 GiB each
    way) through CopyEngine; wall time from submit to CopyHandle.wait(), the
    median of `reps` after one untimed pass.  Also the achievable host link
    (one contiguous 1 GiB copy each way between device and pinned host memory)
    and a pinned host-to-host copy, the reference point for a path with no CPU
    analog.  Returns the result dict (value: harmonic mean of both directions)."""
    import numpy as np
    import torch

    import workloads
    from pipeswift_amd import copy_engine

    L, Pg, P2 = 8, 16384, 8192
    gpu_ids, l2_ids = workloads.config5b_pages(gpu_pages=Pg, l2_pages=P2)
    cache = torch.empty((L, Pg, 2, 16, 8, 128), dtype=torch.bfloat16, device=device)
    cache.view(torch.int16).random_(generator=torch.Generator(device=device).manual_seed(95))
    nbytes = len(gpu_ids) * L * 65536
    results = {}
    for transport in transports:
        eng = copy_engine.CopyEngine([cache], Pg, P2, transport=transport)
        try:
            res = {}
            for direction in ("store", "load"):
                times = []
                for rep in range(reps + 1):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    if direction == "store":
                        h = eng.store(gpu_ids.tolist(), l2_ids.tolist())
                    else:
                        h = eng.load(l2_ids.tolist(), gpu_ids.tolist())
                    h.wait()
                    if rep:
                        times.append(time.perf_counter() - t0)
                res[direction] = {"GB/s": round(nbytes / float(np.median(times)) / 1e9, 2),
                                  "ms": round(1e3 * float(np.median(times)), 3), "runs": h.num_runs * L}
            results[transport] = res
        finally:
            eng.close()
    best = max(results, key=lambda t: min(results[t]["store"]["GB/s"], results[t]["load"]["GB/s"]))
    st, ld = results[best]["store"]["GB/s"], results[best]["load"]["GB/s"]
    value = 2.0 / (1.0 / st + 1.0 / ld)  # both directions, harmonic mean

    del cache
    torch.cuda.empty_cache()
    n = 1 << 30
    dev_buf = torch.empty(n, dtype=torch.uint8, device=device)
    host_a = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    host_b = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    host_a.fill_(3)

    def timed_copy(dst, src, reps=5):
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            dst.copy_(src, non_blocking=True)
            torch.cuda.synchronize()
            t.append(time.perf_counter() - t0)
        return n / float(np.median(t)) / 1e9

    link = {"D2H": timed_copy(host_a, dev_buf), "H2D": timed_copy(dev_buf, host_a)}
    link_hm = 2.0 / (1.0 / link["D2H"] + 1.0 / link["H2D"])
    host_copy = timed_copy(host_b, host_a)
    del dev_buf, host_a, host_b
    torch.cuda.empty_cache()
    blocks_per_s = len(gpu_ids) / ((results[best]["store"]["ms"] + results[best]["load"]["ms"]) / 2e3)
    return {
        "value": round(value, 2), "unit": "GB/s", "steps": reps, "warmup": 1,
        "ms_per_step": results[best]["store"]["ms"] + results[best]["load"]["ms"],
        "blocks_per_s": round(blocks_per_s, 1),
        "config": {"workload": "swap_blocks (config 5b)", "blocks": len(gpu_ids), "layers": L,
                   "bytes_per_block_layer": 65536, "bytes_each_way": nbytes, "transport": best,
                   "all_transports": results},
        "roofline": {"bound": "pcie", "kernel": "blit_pages_kernel" if best == "blit" else best,
                     "achieved": round(value, 2), "peak": 64.0, "unit": "GB/s",
                     "frac": round(value / 64.0, 4), "traffic": None,
                     "achievable": round(link_hm, 2), "frac_of_achievable": round(value / link_hm, 4),
                     "achievable_each_way": {k: round(v, 2) for k, v in link.items()},
                     "achievable_how": "one contiguous 1 GiB copy each way, device <-> pinned host"},
        "cpu_baseline": {"value": round(host_copy, 2), "unit": "GB/s", "cores": 1, "kind": "reference point",
                         "sample": "pinned host-to-host copy of 1 GiB (the swap has no CPU analog)"},
        # The reference publishes one figure at this descriptor size: H2D
        # cuMemcpyBatchAsync at 64 KiB per descriptor on H100 / PCIe Gen5 x16
        # (copy_engine.py:15-21).  Other hardware, so a reference point beside
        # the line, not vs_baseline.
        "vs_published": {"reference_GBps": PUBLISHED_H2D_64K_GBPS, "ours_GBps": ld,
                         "ratio": round(ld / PUBLISHED_H2D_64K_GBPS, 4),
                         "what": "H2D (load) at 64 KiB per descriptor; reference: cuMemcpyBatchAsync on H100, PCIe "
                                 "Gen5 x16, pipeswift/utils/copy_engine.py:15-21"},
    }


def run_swap(args, device):
    res = measure_swap(device, tuple(args.transports.split(",")), args.swap_reps)
    line = dict({"metric": "swap_blocks host-link GB/s (D2H store + H2D load, 4 GiB each way)", "n_gpus": 1,
                 "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bytes",
                 "data": "synthetic (seeded)"}, **res)
    print(json.dumps(line), flush=True)


def run_metadata(args, device):
    res = measure_metadata(device)
    line = dict({"metric": "host us per step for KV metadata (slot_mapping + page_table + H2D)", "n_gpus": 1,
                 "higher_is_better": False, "vs_baseline": None, "dtype": "int64", "data": "synthetic (seeded)"},
                **res)
    print(json.dumps(line), flush=True)


def measure_metadata(device):
    """Host time of one step's KV metadata (prepare_kv_info: slot_mapping,
    page_table, lengths, and their H2D) for config 2 (128 decode sequences,
    contexts up to 32k) and config 3 (6 sequences, 4096 new tokens), against a
    per-token Python restatement of the reference's loop (metadata.py:258-295)."""
    from array import array

    import numpy as np
    import torch

    from oracle import kv_oracle as O
    import workloads
    from pipeswift_amd import metadata

    class Seq:
        def __init__(self, sid, n, off):
            self.seq_id, self.token_ids, self.offset = sid, range(n), off

    cases = {}
    c2 = workloads.config2_fp8_decode()
    cases["config2_decode"] = ([Seq(b, int(c2.extra["ctx"][b]), int(c2.extra["ctx"][b]) - 1) for b in range(128)],
                               {b: array("i", c2.extra["tables"][b].tolist()) for b in range(128)}, True)
    c3 = workloads.config3_chunked()
    cases["config3_chunked"] = ([Seq(b, int(c3.prefix[b] + c3.chunk[b]), int(c3.prefix[b])) for b in range(6)],
                                {b: array("i", c3.block_table[b, : int((c3.prefix[b] + c3.chunk[b] + 15) // 16)]
                                          .tolist()) for b in range(6)}, False)

    def reference_style(seqs, table, ps):
        slot, rows = [], []
        width = max(len(table[s.seq_id]) for s in seqs)
        for s in seqs:
            row = list(table[s.seq_id])
            rows.append(row + [0] * (width - len(row)))
            slot.extend(O.slot_mapping(row, s.offset, len(s.token_ids), ps))
        pt = torch.from_numpy(np.array(rows, dtype=np.int32)).to(device, non_blocking=True)
        sm = torch.from_numpy(np.array(slot, dtype=np.int64)).to(device, non_blocking=True)
        return pt, sm

    out = {}
    for name, (seqs, table, dec) in cases.items():
        for _ in range(5):
            info = metadata.prepare_kv_info(seqs, table, 16, None, None, is_decode=dec, device=device)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        reps = 200
        for _ in range(reps):
            info = metadata.prepare_kv_info(seqs, table, 16, None, None, is_decode=dec, device=device)
        t_ours = (time.perf_counter() - t0) / reps
        torch.cuda.synchronize()
        ref_pt, ref_sm = reference_style(seqs, table, 16)
        torch.cuda.synchronize()
        assert torch.equal(ref_sm, info.slot_mapping) and torch.equal(ref_pt, info.page_table)
        t0 = time.perf_counter()
        rreps = 5
        for _ in range(rreps):
            reference_style(seqs, table, 16)
        t_ref = (time.perf_counter() - t0) / rreps
        out[name] = {"tokens": int(info.slot_mapping.numel()), "pages_wide": int(info.page_table.shape[1]),
                     "ours_us": round(t_ours * 1e6, 1), "reference_style_python_us": round(t_ref * 1e6, 1)}
        progress(f"metadata {name}: ours {out[name]['ours_us']} us, reference-style loop "
                 f"{out[name]['reference_style_python_us']} us")
    out["graph_refresh"] = measure_graph_refresh(device, cases["config2_decode"])
    progress(f"metadata graph_refresh: native {out['graph_refresh']['native']['us']} us, reference-style "
             f"{out['graph_refresh']['reference_style']['us']} us")
    return {"value": out["config3_chunked"]["ours_us"], "unit": "us per step (host)",
            "config": {"workload": "metadata: prepare_kv_info and the graph static refresh", "cases": out},
            "roofline": None,
            "cpu_baseline": {"value": out["config3_chunked"]["reference_style_python_us"], "unit": "us", "cores": 1,
                             "kind": "port", "sample": "per-token Python loop restating metadata.py:258-295"}}


def reference_style_graph_refresh(static, info, cg_bsz, pad_q_len=1):
    """The reference's set_graph_kvcacheinfo (cudagraph.py:75-118) as torch
    device ops, for timing only: five copies, then with a padded batch three
    fills, a zero and the arange chain of the cu_seqlens_q tail."""
    import torch

    bsz, max_pages = info.actual_lens_q.shape[0], info.page_table.shape[1]
    static.page_table[:bsz, :max_pages].copy_(info.page_table, non_blocking=True)
    static.slot_mapping[: info.slot_mapping.shape[0]].copy_(info.slot_mapping, non_blocking=True)
    static.actual_lens_q[:bsz].copy_(info.actual_lens_q, non_blocking=True)
    static.actual_lens_kv[:bsz].copy_(info.actual_lens_kv, non_blocking=True)
    static.cu_seqlens_q[: bsz + 1].copy_(info.cu_seqlens_q, non_blocking=True)
    if bsz != cg_bsz:
        static.actual_lens_q[bsz:].fill_(pad_q_len)
        static.slot_mapping[info.slot_mapping.shape[0]:].fill_(-1)
        static.actual_lens_kv[bsz:].zero_()
        static.page_table[bsz:, :max_pages].zero_()
        tail = static.cu_seqlens_q.shape[0] - bsz
        static.cu_seqlens_q[bsz + 1:].copy_(
            static.cu_seqlens_q[bsz] + torch.arange(pad_q_len, tail * pad_q_len, pad_q_len, dtype=torch.int32,
                                                    device=static.cu_seqlens_q.device), non_blocking=True)


def measure_graph_refresh(device, case, reps=200):
    """Graph static-metadata refresh for config 2's decode batch (128
    sequences, a 1831-page table) into static buffers of a 256-sequence,
    2048-page graph (a padded replay): the native one-launch refresh against
    the reference's copy/fill sequence on the same buffers.  `host_us` is the
    caller's time per call (enqueue only), `us` the time per call with the
    device work included (reps calls, then one synchronize)."""
    import torch

    from pipeswift_amd import cudagraph, metadata

    seqs, table, dec = case
    info = metadata.prepare_kv_info(seqs, table, 16, None, None, is_decode=dec, device=device)
    static = cudagraph.initialize_graph_kvcacheinfo(256, 2048, device=device)
    res = {"batch": len(seqs), "graph_batch": 256, "page_table": list(info.page_table.shape), "static_pages": 2048}
    for name, fn in (("native", cudagraph.set_graph_kvcacheinfo), ("reference_style", reference_style_graph_refresh)):
        for _ in range(10):
            fn(static, info, 256)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn(static, info, 256)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        res[name] = {"host_us": round((t1 - t0) / reps * 1e6, 2), "us": round((t2 - t0) / reps * 1e6, 2)}
    return res


def run_l2_cycle(args, device):
    line = dict({"metric": "L2 offload+restore GB/s through BlockManager (config 5b: 8192 scattered pages of 512 KiB, 4 GiB each way)", "n_gpus": 1, "steps": 1, "warmup": 0, "higher_is_better": True, "scaling": "weak",
                 "vs_baseline": None, "dtype": "bytes", "data": "synthetic (seeded)"}, **measure_l2_cycle(device, 8192))
    print(json.dumps(line), flush=True)


def measure_l2_cycle(device, n=8192):
    """BlockManager's L2 path: an n-page prompt (L=8 layers of [2, 16, 8, 128]
    bf16, 512 KiB per page; n=8192 is config 5b's 4 GiB) is stored to L2, evicted
    from HBM, and restored by a second prompt with the same tokens, on pages
    drawn from seeded shuffles of both free lists (a churned pool, the case the
    deadline is priced for, block_manager.py:646-655).  Reports wall time and
    GB/s of each direction, the deadline the calibrated model set against the
    time the transfer took, host time of the ledger calls, and the restored
    bytes' check.  cpu_baseline: the reference's per-page xxhash loop over the
    same prompt (block_manager.py:678-693) against the native key chain."""
    from array import array
    from collections import deque

    import numpy as np
    import torch

    from oracle import block_ledger as OB
    from pipeswift_amd.block_manager import BlockManager

    class Seq:
        def __init__(self, sid, toks):
            self.seq_id, self.token_ids, self.offset = sid, array("i", toks), 0
            self.finished, self.l2_load_pending, self.page_hashes, self.l2_probe_resume = False, False, None, None

    L, ps = 8, 16
    P = n + 2
    cache = torch.zeros((L, P, 2, ps, 8, 128), dtype=torch.bfloat16, device=device)
    page_bytes = L * 2 * ps * 8 * 128 * 2
    t0 = time.perf_counter()
    with warnings.catch_warnings():  # L2 holds n of the n + 2 GPU pages, by design of this cycle
        warnings.simplefilter("ignore", RuntimeWarning)
        m = BlockManager(P, ps, [cache[:, :, 0], cache[:, :, 1]], None, kv_cache_tensor=cache,
                         l2_cache_gb=n * page_bytes / 1024**3)
    t_init = time.perf_counter() - t0
    rng = np.random.default_rng(1005)
    m.free_page_queue = deque(int(x) for x in rng.permutation(np.arange(1, P)))
    m.l2_pool.free_page_queue = deque(int(x) for x in rng.permutation(n))
    prompt = rng.integers(0, 150000, n * ps + 1).tolist()
    a = Seq(1, prompt)
    t0 = time.perf_counter()
    m.allocate_prefill(a)
    t_alloc = time.perf_counter() - t0
    table_a = torch.tensor(list(m.kv_page_table[1])[:n], dtype=torch.int64, device=device)
    flat = cache.view(torch.int16)
    for l in range(L):  # page j of the prompt holds the value j + l everywhere
        for j0 in range(0, n, 512):
            idx = table_a[j0:j0 + 512]
            v = (torch.arange(j0, j0 + len(idx), device=device, dtype=torch.int16) + l).view(-1, 1, 1, 1, 1)
            flat[l].index_copy_(0, idx, v.expand(len(idx), 2, ps, 8, 128).contiguous())
    torch.cuda.synchronize()
    res = {"init_s (incl. calibrate)": round(t_init, 3), "cost_model": m.l2_cost_model, "views": m.l2_views,
           "page_bytes": page_bytes, "pages": n}

    m.poll_l2_events(0)
    t0 = time.perf_counter()
    m.schedule_l2_stores_for_confirmed_seq(a)
    t_sched = time.perf_counter() - t0
    st = m.pending_l2_stores[-1]
    st.copy.wait()
    t_store = time.perf_counter() - t0
    owed_store = m._l2_owed_s["store"] - 1 * m.l2_step_ms / 1000
    res["store"] = {"GB/s": n * page_bytes / t_store / 1e9, "wall_ms": 1e3 * t_store,
                    "host_schedule_ms": 1e3 * t_sched, "runs": st.copy.num_runs,
                    "predicted_ms": 1e3 * owed_store, "due_step": st.due_step}
    m.poll_l2_events(st.due_step)
    m.deallocate(a)
    filler = Seq(2, [7] * (ps * (P - 1)))
    m.allocate_prefill(filler)
    m.deallocate(filler)

    b = Seq(3, prompt)
    step = m.l2_step
    t0 = time.perf_counter()
    m.allocate_prefill(b)
    t_alloc_b = time.perf_counter() - t0
    m.flush_l2_loads()
    t_flush = time.perf_counter() - t0
    groups = list(m.pending_l2_loads)
    for g in groups:
        g.copy.wait()
    t_load = time.perf_counter() - t0
    owed_load = m._l2_owed_s["load"] - step * m.l2_step_ms / 1000
    m.poll_l2_events(groups[-1].due_step)
    assert not b.l2_load_pending and b.offset == n * ps
    table_b = torch.tensor(list(m.kv_page_table[3])[:n], dtype=torch.int64, device=device)
    ok = True
    for l in range(L):
        for j0 in range(0, n, 512):
            got = flat[l].index_select(0, table_b[j0:j0 + 512])
            want = (torch.arange(j0, j0 + got.shape[0], device=device, dtype=torch.int16) + l).view(-1, 1, 1, 1, 1)
            ok = ok and bool((got == want).all())
    assert ok, "restored pages differ"
    res["restore"] = {"GB/s": n * page_bytes / t_load / 1e9, "wall_ms": 1e3 * t_load,
                      "host_allocate_prefill_ms": 1e3 * t_alloc_b, "host_flush_ms": 1e3 * (t_flush - t_alloc_b),
                      "transfers": len(groups), "runs": sum(g.copy.num_runs for g in groups),
                      "predicted_ms": 1e3 * owed_load, "last_due_step": groups[-1].due_step - step}
    res["bytes_checked"] = True

    # host cost of keying the prompt: native chain against the reference's loop
    # both timed with the cyclic collector off (after one collection), so that a
    # collection pass over the process's objects lands in neither
    import gc

    reps = 20
    seqs = [Seq(9, prompt) for _ in range(reps + 1)]  # fresh sequences: the keys are memoized per sequence
    oracle_ledger = OB.RefLedger(4, ps)
    gc.collect()
    gc.disable()
    try:
        t0 = time.perf_counter()
        for sq in seqs[:reps]:
            m._prompt_page_hashes(sq)
        t_native = (time.perf_counter() - t0) / reps
        t0 = time.perf_counter()
        ref_keys = oracle_ledger.prompt_pages(seqs[reps])
        t_ref = time.perf_counter() - t0
    finally:
        gc.enable()
    assert [h for h, _ in ref_keys] == [h for h, _ in m._prompt_page_hashes(Seq(9, prompt))]
    res["prompt_keys_ms"] = {"native": 1e3 * t_native, "reference_loop": 1e3 * t_ref, "first_prefill_ms": 1e3 * t_alloc}
    stg, ldg = res["store"]["GB/s"], res["restore"]["GB/s"]
    progress(f"l2_cycle {n} pages: store {stg:.2f} GB/s in {res['store']['wall_ms']:.1f} ms (deadline model "
             f"{res['store']['predicted_ms']:.1f} ms), restore {ldg:.2f} GB/s in {res['restore']['wall_ms']:.1f} ms "
             f"(model {res['restore']['predicted_ms']:.1f} ms)")
    value = 2.0 / (1.0 / stg + 1.0 / ldg)
    m.l2_copy_engine.close()
    del m, cache
    torch.cuda.empty_cache()
    return {
        "value": round(value, 2), "unit": "GB/s",
        "ms_per_step": res["store"]["wall_ms"] + res["restore"]["wall_ms"],
        "config": {"workload": f"l2_cycle: store -> evict -> restore of a {n}-page prompt through BlockManager",
                   "results": res},
        "roofline": {"bound": "pcie", "achieved": round(value, 2), "peak": 64.0, "unit": "GB/s",
                     "frac": round(value / 64.0, 4), "traffic": None},
        "cpu_baseline": {"value": round(1e3 * t_ref, 2), "unit": f"ms to key the {n}-page prompt", "cores": 1,
                         "kind": "port", "sample": "per-page xxhash loop of block_manager.py:678-693 (oracle), "
                                                   f"native key chain {1e3 * t_native:.2f} ms"},
    }


def run_attention_shapes(args, device):
    """Decode attention over several batch shapes and block sizes, under the
    balanced schedule (num_splits 0, the default) and under the split schedule
    at the count the split heuristic would pick; random FP8 pages, shuffled
    block tables.  `us`
    is the device time per call, from HIP events around graph replays of 10
    calls; `eager_us` is the same around eager calls, which includes the host
    time of the Python call where that exceeds the device time."""
    import math

    import numpy as np
    import torch

    from pipeswift_amd import attention

    rng = np.random.default_rng(0)
    shapes = [
        ("1 x 131072, 4 kv heads, group 8", 4, 8, [131072]),
        ("1 x 32768", 8, 4, [32768]),
        ("8 x 32768", 8, 4, [32768] * 8),
        ("32 x 8192", 8, 4, [8192] * 32),
        ("128 log-uniform 128-32768", 8, 4, [int(x) for x in np.exp(rng.uniform(np.log(128), np.log(32768), 128))]),
        ("64 uniform 1-4096", 8, 4, [int(x) for x in rng.integers(1, 4096, 64)]),
    ]
    # group 8 (64 query heads over 8 kv heads, Llama-3-70B class) on two of them
    shapes += [("128 log-uniform 128-32768, group 8", 8, 8, shapes[4][3]), ("32 x 8192, group 8", 8, 8, [8192] * 32)]
    shapes = [(*x, 16) for x in shapes]
    # pages that are not a power of two >= 16: the general-page kernel variants
    shapes += [("128 log-uniform 128-32768, pages of 24", 8, 4, shapes[4][3], 24),
               ("32 x 8192, pages of 48", 8, 4, [8192] * 32, 48), ("32 x 8192, pages of 5", 8, 4, [8192] * 32, 5),
               ("32 x 8192, group 8, pages of 24", 8, 8, [8192] * 32, 24), ("1 x 32768, pages of 24", 8, 4, [32768], 24)]
    reps = max(10, min(args.steps, 50))
    results = []
    for name, Hkv, G, lens, ps in shapes:
        B = len(lens)
        g = torch.Generator(device=device).manual_seed(1)
        pages = [math.ceil(x / ps) for x in lens]
        P = sum(pages) + 8
        cache = torch.empty(P, 2, ps, Hkv, 128, dtype=torch.float8_e4m3fn, device=device)
        cache.view(torch.uint8).random_(0, 120, generator=g)
        W = max(pages)
        bt = torch.zeros(B, W, dtype=torch.int32)
        perm = torch.randperm(P, generator=torch.Generator().manual_seed(2))
        o = 0
        for b in range(B):
            bt[b, : pages[b]] = perm[o: o + pages[b]].to(torch.int32)
            o += pages[b]
        bt = bt.to(device)
        sl = torch.tensor(lens, dtype=torch.int32, device=device)
        q = torch.randn(B, Hkv * G, 128, device=device, generator=g).to(torch.bfloat16)
        out = torch.empty(B, Hkv * G, 128, dtype=torch.bfloat16, device=device)
        kv_bytes = sum(lens) * Hkv * 128 * 2
        split = min(128, max(20, math.ceil(1536 / (B * Hkv))))
        row = {"shape": name, "block_size": ps, "tokens": sum(lens), "kv_bytes": kv_bytes}
        for label, ns in (("balanced", 0), (f"split_{split}", split)):
            ws = torch.empty(attention.workspace_floats(B, Hkv * G, Hkv, W * ps, ns), dtype=torch.float32, device=device)

            def call():
                attention.paged_decode_attention(q, cache[:, 0], cache[:, 1], bt, sl, None, out=out, workspace=ws,
                                                 num_splits=ns)

            stream = torch.cuda.Stream(device)
            with torch.cuda.stream(stream):
                for _ in range(5):
                    call()
                stream.synchronize()
                # eager: host time per call included (small shapes are host bound)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    call()
                e1.record(stream)
                torch.cuda.synchronize()
                eager_us = e0.elapsed_time(e1) / reps * 1e3
                # graph replay: the device time per call
                per_graph = 10
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for _ in range(per_graph):
                        call()
                graph.replay()
                stream.synchronize()
                n_rep = max(1, reps // per_graph)
                e0.record(stream)
                for _ in range(n_rep):
                    graph.replay()
                e1.record(stream)
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) / (n_rep * per_graph) * 1e3
                del graph
            row[label] = {"us": round(us, 2), "GB/s": round(kv_bytes / us / 1e3, 1), "eager_us": round(eager_us, 2)}
        results.append(row)
        progress("attention_shapes " + ", ".join(f"{k}={v}" for k, v in row.items()))
    print(json.dumps({"metric": "decode attention us per call, balanced vs split schedule", "unit": "us",
                      "calls_per_shape": reps, "shapes": results}), flush=True)


def run_swap_sweep(args, device):
    """Host-link GB/s against bytes per page at a fixed 256 MiB per transfer,
    scattered pages (every page its own run), both directions, per transport:
    the MI355X counterpart of the descriptor-size table in copy_engine.py:15-21.
    `*_GBs` is submit-to-completion wall time (host coalescing included);
    `*_gpu_GBs` is HIP-event time on the copy stream."""
    import numpy as np
    import torch

    from pipeswift_amd import copy_engine

    total = 256 << 20
    rows = []
    for page in (4096, 8192, 16384, 32768, 65536, 131072, 262144, 524288):
        n = total // page
        cache = torch.empty((1, n + 1, page), dtype=torch.uint8, device=device)
        rng = np.random.default_rng(page)
        gpu_ids = rng.permutation(n + 1)[:n]
        l2_ids = rng.permutation(n)
        row = {"bytes_per_page": page}
        for transport in args.transports.split(","):
            eng = copy_engine.CopyEngine([cache], n + 1, n, transport=transport, timing_events=True)
            try:
                for direction in ("store", "load"):
                    times, gpu_times = [], []
                    params = eng.store_params if direction == "store" else eng.load_params
                    for rep in range(3):
                        torch.cuda.synchronize()
                        start = torch.cuda.Event(enable_timing=True)
                        start.record(params.stream)  # ahead of the copy thread's work on that stream
                        t0 = time.perf_counter()
                        h = eng.store(gpu_ids, l2_ids) if direction == "store" else eng.load(l2_ids, gpu_ids)
                        h.wait()
                        if rep:
                            times.append(time.perf_counter() - t0)
                            gpu_times.append(start.elapsed_time(h.event) / 1e3)
                    row[f"{transport}_{direction}_GBs"] = round(total / min(times) / 1e9, 2)
                    row[f"{transport}_{direction}_gpu_GBs"] = round(total / min(gpu_times) / 1e9, 2)
            finally:
                eng.close()
        rows.append(row)
        progress("swap_sweep " + ", ".join(f"{k}={v}" for k, v in row.items()))
    best = max(min(r[f"{t}_{d}_GBs"] for d in ("store", "load")) for r in rows for t in args.transports.split(","))
    line = {"metric": "host-link GB/s vs bytes per page (256 MiB scattered transfer)", "value": best, "unit": "GB/s",
            "n_gpus": 1, "higher_is_better": True, "vs_baseline": None, "dtype": "bytes", "data": "synthetic",
            "config": {"workload": "swap_sweep", "rows": rows},
            "roofline": {"bound": "pcie", "achieved": best, "peak": 64.0, "unit": "GB/s", "frac": round(best / 64.0, 4),
                         "traffic": None}}
    print(json.dumps(line), flush=True)


# --------------------------------------------------------------------------- #
# CPU baseline: the numpy oracle on a bounded sample of the same workload
# --------------------------------------------------------------------------- #


def _raw(t):
    import numpy as np
    import torch

    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def cpu_decode_attention(kc, vc, bt, ctx, q, scales, kv_bytes, budget_s=10.0, q_len=1):
    """The float64 numpy oracle over the first sequences of the batch (q_len
    causal query tokens each) until the budget is spent; returns (fraction of
    one launch's K/V bytes processed, seconds, sample)."""
    import numpy as np

    from oracle import kv_oracle as O

    ks, vs = (float(x) for x in scales.cpu())
    t0 = time.perf_counter()
    done = 0
    nbytes = 0
    H, D = kc.shape[2], kc.shape[3]
    while time.perf_counter() - t0 < budget_s and done < len(ctx):
        n = int(ctx[done])
        w = (n + 15) // 16
        pages = bt[done, :w].long()
        k = _raw(kc[pages].cpu())
        v = _raw(vc[pages].cpu())
        O.paged_decode_attention(_raw(q[done * q_len: (done + 1) * q_len].cpu()), "bf16", k, v,
                                 np.arange(w, dtype=np.int32)[None], [n], D ** -0.5, None,
                                 np.full((1, H), ks, np.float32), np.full((1, H), vs, np.float32),
                                 cu_seqlens_q=[0, q_len], causal=True)
        nbytes += n * H * D * 2
        done += 1
    el = time.perf_counter() - t0
    return nbytes / kv_bytes, el, f"float64 numpy oracle over the first {done} of 128 sequences"


def torch_cpu_decode_attention_step(kc, vc, bt, ctx, q, scales, q_len=1, max_seqs=16):
    """torch on the host for the decode attention: the first `max_seqs`
    sequences' FP8 pages are copied to host memory once; a step dequantizes
    them (x * descale, fp32) and computes causal softmax(Q K^T / sqrt(D)) V for
    each kv head's query group.  Returns (step, outputs, sample bytes): outputs
    holds each sequence's fp32 [q_len, Hq, D] after a step; sample bytes are
    the algorithmic bytes of those sequences (K/V rows, page ids, queries and
    outputs)."""
    import torch

    ks, vs = (float(x) for x in scales.cpu())
    H, D = kc.shape[2], kc.shape[3]
    Hq = q.shape[1]
    G = Hq // H
    seqs, sample_bytes = [], 0
    for b in range(min(max_seqs, len(ctx))):
        n = int(ctx[b])
        pages = bt[b, : (n + 15) // 16].long()
        seqs.append((kc[pages].cpu(), vc[pages].cpu(), q[b * q_len: (b + 1) * q_len].cpu(), n))
        sample_bytes += n * H * D * 2 + pages.numel() * 4 + 2 * q_len * Hq * D * 2
    scale = D ** -0.5
    outs = [None] * len(seqs)

    def step():
        for i, (k8, v8, qb, n) in enumerate(seqs):
            k = k8.float().reshape(-1, H, D)[:n].mul_(ks).permute(1, 2, 0)  # [H, D, n]
            v = v8.float().reshape(-1, H, D)[:n].mul_(vs).transpose(0, 1)  # [H, n, D]
            qf = qb.float().view(q_len, H, G, D).permute(1, 0, 2, 3).reshape(H, q_len * G, D)
            s = torch.matmul(qf, k) * scale  # [H, q_len * G, n]
            if q_len > 1:  # query row r sees keys 0 .. n - q_len + r
                row = torch.arange(q_len).repeat_interleave(G).view(1, -1, 1)
                s = s.masked_fill(torch.arange(n).view(1, 1, -1) > (n - q_len + row), float("-inf"))
            o = torch.matmul(torch.softmax(s, -1), v)  # [H, q_len * G, D]
            outs[i] = o.view(H, q_len, G, D).permute(1, 0, 2, 3).reshape(q_len, Hq, D)

    return step, outs, sample_bytes


def torch_cpu_decode_attention(kc, vc, bt, ctx, q, scales, full_bytes, budget_s=3.0, q_len=1):
    """Times torch_cpu_decode_attention_step; returns (launch equivalents,
    seconds): steps scaled by the sample's share of one launch's bytes."""
    step, _, sample_bytes = torch_cpu_decode_attention_step(kc, vc, bt, ctx, q, scales, q_len)
    n, el = _timed(step, budget_s)
    return n * sample_bytes / full_bytes, el


def cpu_append(case, fp8, budget_s=10.0):
    import numpy as np

    from oracle import kv_oracle as O

    key, value = _raw(case.key()), _raw(case.value())
    cache = np.zeros(tuple(case.cache.shape), np.uint8 if fp8 else np.uint16)
    slots = case.slot_mapping.numpy()
    ks = vs = None
    if fp8:
        ks, _ = O.amax_scale(key, "bf16")
        vs, _ = O.amax_scale(value, "bf16")
    n = 0
    t0 = time.perf_counter()
    while True:
        O.reshape_and_cache(key, value, cache[:, 0], cache[:, 1], slots, "bf16", "fp8" if fp8 else "bf16", ks, vs)
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= 20000:
            break
    return n, el, f"{n} steps of the numpy oracle append (same inputs and cache geometry)"


def cpu_mla_fp8_tiles(case, budget_s=10.0):
    from oracle import kv_oracle as O

    kv_c, k_pe = _raw(case.kv_c), _raw(case.k_pe())
    cache = _raw(case.cache).copy()
    slots = case.slot_mapping.numpy()
    n = 0
    t0 = time.perf_counter()
    while True:
        O.concat_and_cache_mla_tiles(kv_c, k_pe, cache, slots)
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            break
    return n, el, f"{n} steps of the numpy oracle tile-scaled FP8 MLA append (same inputs and cache)"


def cpu_gather(cc, budget_s=10.0):
    from oracle import kv_oracle as O

    kc = _raw(cc.append.cache[:, 0])
    n = 0
    t0 = time.perf_counter()
    while True:
        O.gather_cache(kc, cc.block_table.numpy(), cc.cu_seq_lens.numpy())
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            break
    # the oracle gathered K only; the GPU step moves K and V
    return n / 2.0, el, f"{n} K-only numpy oracle gathers (counted as {n / 2:.1f} K+V steps)"


def _timed(fn, budget_s):
    n = 0
    t0 = time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            return n, el


def torch_cpu_append_step(case, fp8):
    """The reference's CPU path for the append (as the north star names it): torch
    index_put_ of the valid tokens' K and V rows into host caches of the same
    strided [P, 2, ps, H, D] layout, after fp8_kv.quantize (fp8_kv.py:75-77,
    x / scale clamped to +-448, then float8_e4m3fn) for an FP8 cache.  Returns
    (step, cache)."""
    import torch

    key, value = case.key(), case.value()
    slots = case.slot_mapping
    valid = slots >= 0
    ps = case.cache.shape[2]
    blk, off = slots[valid] // ps, slots[valid] % ps
    kv, vv = key[valid], value[valid]
    cache = torch.zeros(tuple(case.cache.shape), dtype=torch.float8_e4m3fn if fp8 else torch.bfloat16)
    kc, vc = cache[:, 0], cache[:, 1]
    ks = vs = None
    if fp8:
        from oracle import kv_oracle as O

        ks, _ = O.amax_scale(_raw(key), "bf16")
        vs, _ = O.amax_scale(_raw(value), "bf16")

    def step():
        if fp8:
            kc.index_put_((blk, off), (kv.float() / ks).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
            vc.index_put_((blk, off), (vv.float() / vs).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
        else:
            kc.index_put_((blk, off), kv)
            vc.index_put_((blk, off), vv)

    return step, cache


def torch_cpu_append(case, fp8, budget_s=3.0, rescale=False):
    """The torch host append.  ``rescale``: each step first recomputes the two
    per-tensor scales (torch amax of |K| and |V| over 448), as the GPU step
    of fp8_decode_write does."""
    import torch

    step, _ = torch_cpu_append_step(case, fp8)
    if not rescale:
        return _timed(step, budget_s)
    key, value = case.key(), case.value()

    def full():
        (key.float().abs().amax() / 448.0).item(), (value.float().abs().amax() / 448.0).item()
        step()

    return _timed(full, budget_s)


def torch_cpu_kv_scales(case, budget_s=3.0):
    """torch on the host for the per-tensor scales: amax of |K| and of |V| in
    fp32, each divided by 448."""
    key, value = case.key(), case.value()

    def step():
        return key.float().abs().amax() / 448.0, value.float().abs().amax() / 448.0

    return _timed(step, budget_s)


def torch_cpu_mla_step(case, scale):
    """torch on the host for the MLA append: the [kv_c | k_pe] rows of the
    valid tokens index_put_ into a [P, ps, 576] host cache, quantized first as
    fp8_kv.quantize does (x / scale clamped to +-448, float8_e4m3fn) when
    ``scale`` is given.  Returns (step, cache)."""
    import torch

    slots = case.slot_mapping
    ps = case.cache.shape[1]
    valid = slots >= 0
    blk, off = slots[valid] // ps, slots[valid] % ps
    rows = torch.cat([case.kv_c, case.k_pe()], 1)[valid]
    cache = torch.zeros(tuple(case.cache.shape), dtype=torch.float8_e4m3fn if scale is not None else torch.bfloat16)

    def step():
        if scale is not None:
            cache.index_put_((blk, off), (rows.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
        else:
            cache.index_put_((blk, off), rows)

    return step, cache


def torch_cpu_mla(case, scale, budget_s=3.0):
    step, _ = torch_cpu_mla_step(case, scale)
    return _timed(step, budget_s)


def torch_cpu_gather_step(cc):
    """torch on the host for the gather: index_select of each sequence's pages of
    the K and V caches, reshaped to rows and cut to the sequence's tokens.
    Returns (step, outputs), outputs filled by the last step as [K rows, V rows]."""
    import torch

    kc, vc = cc.append.cache[:, 0], cc.append.cache[:, 1]
    cu = cc.cu_seq_lens.tolist()
    ps = kc.shape[1]
    tables = []
    for b in range(len(cu) - 1):
        n = cu[b + 1] - cu[b]
        tables.append((cc.block_table[b, : (n + ps - 1) // ps].long(), n))
    out = [None, None]

    def step():
        k_rows, v_rows = [], []
        for t, n in tables:
            k_rows.append(torch.index_select(kc, 0, t).reshape(-1, *kc.shape[2:])[:n])
            v_rows.append(torch.index_select(vc, 0, t).reshape(-1, *vc.shape[2:])[:n])
        out[0], out[1] = torch.cat(k_rows), torch.cat(v_rows)

    return step, out


def torch_cpu_gather(cc, budget_s=3.0):
    step, _ = torch_cpu_gather_step(cc)
    return _timed(step, budget_s)


def _copy_blocks_sample(P=256, n=128, L=61):
    """A bounded host sample of config 5a: L layers of P 64 KiB blocks, n disjoint
    pairs (about 1 GiB of host stack, 0.5 GB moved per step)."""
    import torch

    g = torch.Generator().manual_seed(1005)
    stack = torch.randint(-32768, 32767, (L, P, 2, 16, 8, 128), generator=g, dtype=torch.int16)
    perm = torch.randperm(P, generator=g)
    pairs = torch.stack([perm[:n], perm[n: 2 * n]], 1)
    moved = L * n * 65536 * 2 + n * 16
    return stack, pairs, moved


def cpu_copy_blocks(full_bytes, budget_s=10.0):
    from oracle import kv_oracle as O

    stack, pairs, moved = _copy_blocks_sample()
    st, m = stack.numpy(), pairs.numpy()
    n, el = _timed(lambda: O.copy_blocks(st, m), budget_s)
    return n * moved / full_bytes, el, (f"{n} numpy oracle snapshot copies of 128 pairs x 61 layers of a 256-block "
                                        f"host stack ({moved / 1e9:.2f} GB each), scaled to config 5a's bytes")


def torch_cpu_copy_blocks(full_bytes, budget_s=3.0):
    """The host path the survey names for copy_blocks: a snapshot index copy
    stack[:, dst] = stack[:, src].clone() on a bounded sample."""
    stack, pairs, moved = _copy_blocks_sample()
    src, dst = pairs[:, 0], pairs[:, 1]

    def step():
        stack[:, dst] = stack[:, src].clone()

    n, el = _timed(step, budget_s)
    return n * moved / full_bytes, el


# --------------------------------------------------------------------------- #
# timing
# --------------------------------------------------------------------------- #


def launch_sets(steps, rotate):
    """Rotation set of each of the `steps` timed launches, in order: exactly
    `steps` entries cycling through the `rotate` input sets."""
    R = max(1, int(rotate))
    return [i % R for i in range(max(0, int(steps)))]


_SPIN_US_PER_CYCLE = None


def _spin_us_per_cycle(device):
    """Microseconds per cycle of torch's spin kernel on this GPU, measured once."""
    global _SPIN_US_PER_CYCLE
    import torch

    if _SPIN_US_PER_CYCLE is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(100_000)
        e0.record()
        torch.cuda._sleep(SPIN_CYCLES)
        e1.record()
        torch.cuda.synchronize()
        _SPIN_US_PER_CYCLE = e0.elapsed_time(e1) * 1e3 / SPIN_CYCLES
    return _SPIN_US_PER_CYCLE


def time_launches(launch, rotate, steps, warmup, device, eager_calls=200, eager=False):
    """HIP-event time of exactly `steps` launches on one stream, after `warmup`
    untimed ones.  Launch i uses rotation set i % rotate.

    Up to QUEUED_MAX launches ("queued"): a spin kernel is enqueued first, long
    enough to cover the host's enqueue time of the K launches (twice the
    measured per-call host time, plus 0.2 ms), then the start event, the K
    launches and the end event.  The GPU reaches the start event only after
    the spin, by which time all K launches wait in the queue, so the events
    bracket K back-to-back kernels.  That is checked: the host's enqueue
    interval (from before the spin to after the end event) must be shorter
    than the GPU's interval from an event before the spin to the start event;
    otherwise the spin doubles (three attempts) and the graph method is used.

    Longer runs ("graph"): the K launches are captured into one graph, replayed
    once untimed (the first replay also uploads the graph), and stream events
    bracket a second replay, which includes the replay's own fixed cost (about
    15 us; torch refuses timing events inside a graph on ROCm, and HIP's
    external event-record node fails under capture on this runtime).  Graph
    replay is how the reference runs its decode step (llm.py:634-681), and a
    replayed dispatch costs less than a queued one.
    `eager` times plain launches between the events, without a spin
    ("eager": the host's launch rate included).

    Returns a dict with the elapsed ms, the launch count, the method and the
    host wall time of one eager call (Python shim, argument checks, launch)."""
    import torch

    R = max(1, int(rotate))
    sets = launch_sets(steps, R)
    stream = torch.cuda.Stream(device)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(min(R, 8)):
            launch(i)  # eager warmup of every code path before capture
        for i in range(warmup):
            launch(i % R)
        stream.synchronize()
        # host wall time per eager call (Python shim, argument checks, launch):
        # what a caller that does not capture graphs pays, and what the queued
        # method's spin has to cover
        eager_n = max(1, min(eager_calls, steps))
        t0 = time.perf_counter()
        for i in range(eager_n):
            launch(i % R)
        stream.synchronize()
        eager_us = (time.perf_counter() - t0) / eager_n * 1e6
    torch.cuda.synchronize()

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    method, ms = None, None
    if not eager and 0 < steps <= QUEUED_MAX:
        us_per_cycle = _spin_us_per_cycle(device)
        spin_us = 2.0 * steps * eager_us + 200.0
        for _ in range(3):
            cycles = int(spin_us / us_per_cycle)
            with torch.cuda.stream(stream):
                h0 = time.perf_counter()
                ev[0].record(stream)
                torch.cuda._sleep(cycles)
                ev[1].record(stream)
                for i in sets:
                    launch(i)
                ev[2].record(stream)
                h1 = time.perf_counter()
            torch.cuda.synchronize()
            if (h1 - h0) * 1e3 < ev[0].elapsed_time(ev[1]):
                method, ms = "queued", ev[1].elapsed_time(ev[2])
                break
            spin_us *= 2.0
    if method is None and not eager and steps > 0:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for i in sets:
                    launch(i)
            graph.replay()  # untimed: the first replay also uploads the graph
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)  # keeps host submission out of the timed region
            ev[1].record(stream)
            graph.replay()
            ev[2].record(stream)
        torch.cuda.synchronize()
        method, ms = "graph", ev[1].elapsed_time(ev[2])
        del graph
    if method is None:
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)
            ev[1].record(stream)
            for i in sets:
                launch(i)
            ev[2].record(stream)
        torch.cuda.synchronize()
        method, ms = "eager", ev[1].elapsed_time(ev[2])
    how = {"queued": "HIP stream events around K back-to-back launches already queued behind a spin kernel",
           "graph": "HIP stream events around one (warm) graph replay of the K launches",
           "eager": "HIP stream events around K eager launches"}[method]
    return {"ms": ms, "launches": len(sets), "method": method, "timing": how, "eager_us": eager_us}


SETUPS = {
    "fp8_decode_append": lambda a, d: setup_append(a, d, fp8=True),
    "fp8_decode_write": lambda a, d: setup_append(a, d, fp8=True, rescale=True),
    "bf16_append": lambda a, d: setup_append(a, d, fp8=False),
    "kv_scales": setup_kv_scales,
    "decode_attention": setup_decode_attention,
    "decode_attention_q4": lambda a, d: setup_decode_attention(a, d, q_len=4),
    "prefill_attention": setup_prefill_attention,
    "fp8_prefill_append": lambda a, d: setup_prefill_append(a, d, tokens=a.tokens or 32768, fp8=True),
    "bf16_prefill_append": lambda a, d: setup_prefill_append(a, d, tokens=a.tokens or 32768, fp8=False),
    "chunked_append": lambda a, d: setup_chunked(a, d, gather=False),
    "gather": lambda a, d: setup_chunked(a, d, gather=True),
    "mla_prefill": lambda a, d: setup_mla(a, d, decode=False),
    "mla_decode": lambda a, d: setup_mla(a, d, decode=True),
    "mla_prefill_fp8": lambda a, d: setup_mla(a, d, decode=False, fp8=True),
    "mla_decode_fp8": lambda a, d: setup_mla(a, d, decode=True, fp8=True),
    "mla_fp8_tiles_prefill": lambda a, d: setup_mla_fp8_tiles(a, d, decode=False),
    "mla_fp8_tiles_decode": lambda a, d: setup_mla_fp8_tiles(a, d, decode=True),
    "copy_blocks": setup_copy_blocks,
}

# The default run: config 2 is the headline (`value`); every other benchmark
# configuration gets a bounded run of its own under `secondary`, each timed
# the same way (exactly `steps` launches after `warmup`), with CPU baselines
# on a short budget.  (name, steps, warmup)
SECONDARY = (
    ("decode_attention", 256, 8),
    ("decode_attention_q4", 256, 8),
    ("fp8_prefill_append", 256, 16),
    ("fp8_decode_write", 1024, 64),
    ("kv_scales", 1024, 64),
    ("bf16_append", 1024, 64),
    ("chunked_append", 1024, 64),
    ("gather", 64, 8),
    ("mla_prefill", 1024, 64),
    ("mla_decode", 1024, 64),
    ("mla_prefill_fp8", 1024, 64),
    ("mla_decode_fp8", 1024, 64),
    ("copy_blocks", 8, 2),
    ("swap", 2, 1),
    ("l2_cycle", 2048, 0),  # (name, pages, -): the BlockManager store -> evict -> restore cycle, 1 GiB each way
    ("prefill_attention", 16, 2),
    ("metadata", 0, 0),
)


def _load_traffic():
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    return {}


def measure_workload(args, device, name, steps, warmup, achievable, cpu_budget, port_budget, copy_floor=True):
    """Set up one workload, time exactly `steps` launches and return its result
    dict (value, roofline, CPU baselines); frees its device memory on return."""
    import gc

    import torch

    launch, info = SETUPS[name](args, device)
    R = info.get("rotate", args.rotate)
    t = time_launches(launch, R, steps, warmup, device, eager=args.eager)
    per_launch_s = t["ms"] / 1e3 / t["launches"]
    achieved = info["bytes"] / per_launch_s / 1e9
    # For the microsecond workloads the same kernel is also timed over 2048
    # launches in one graph: the per-launch time inside a long graph, such as
    # a decode step, a cross-check of the short run's method.
    steady = None
    if not args.eager and steps < STEADY_STEPS and info["bytes"] < (64 << 20):
        ts = time_launches(launch, R, STEADY_STEPS, warmup, device, eager_calls=1)
        steady = ts["ms"] * 1e3 / ts["launches"]
    floor = None
    if copy_floor and info["bytes"] < (64 << 20):
        floor = measure_copy_floor(device, info["bytes"], steps)
    traffic = _load_traffic().get(name, {}).get("bytes_per_launch")

    cpu_oracle = None
    threads0 = torch.get_num_threads()
    if port_budget > 0 and info.get("cpu") is not None:
        torch.set_num_threads(1)
        n, el, sample = info["cpu"](port_budget)
        cpu_oracle = {"value": round(info["bytes"] * n / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                      "sample": f"{sample}; {el:.1f} s on 1 thread",
                      "tokens_per_s": round(info["tokens"] * n / el, 1)}
    cpu = None
    if cpu_budget > 0 and info.get("cpu_torch") is not None:
        threads = _cpu_threads()
        torch.set_num_threads(threads)
        n, el = info["cpu_torch"](cpu_budget)
        torch.set_num_threads(1)
        n1, el1 = info["cpu_torch"](cpu_budget)
        # per launch: bytes (GB/s) or, for a matrix-core-bound workload, FLOPs (TFLOP/s)
        work, div, unit = (info["flops"], 1e12, "TFLOP/s") if info.get("flops") else (info["bytes"], 1e9, "GB/s")
        cpu = {"value": round(work * n / el / div, 4), "unit": unit, "cores": threads, "kind": "port",
               "value_1thread": round(work * n1 / el1 / div, 4),
               "tokens_per_s": round(info["tokens"] * n / el, 1),
               "sample": f"{info.get('cpu_torch_what', 'torch on host tensors of the same layout')}: "
                         f"{n:.3g} steps in {el:.1f} s on {threads} threads, {n1:.3g} in {el1:.1f} s on 1"}
    torch.set_num_threads(threads0)
    res = {
        "value": round(achieved, 2),
        "unit": "GB/s",
        "steps": t["launches"],
        "warmup": warmup,
        "ms_per_step": t["ms"] / t["launches"],
        "tokens_per_s": round(info["tokens"] / per_launch_s, 1),
        "pct_of_peak": round(100.0 * achieved / PEAK_HBM_GBS, 3),
        "dtype": info["dtype"],
        "config": dict(info["config"], rotation_sets=R, timing=t["timing"]),
        "roofline": {
            "bound": "hbm",
            "kernel": info["kernel"],
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 5),
            "bytes_per_launch": info["bytes"],
            "us_per_launch": round(per_launch_s * 1e6, 3),
            "steady_us_per_launch": None if steady is None else round(steady, 3),
            "steady_frac": None if steady is None else round(info["bytes"] / steady / 1e3 / PEAK_HBM_GBS, 5),
            "traffic": traffic,
            "achievable": None if achievable is None else round(achievable, 1),
            "frac_of_achievable": None if achievable is None else round(achieved / achievable, 5),
        },
        "copy_floor": None if floor is None else {
            "us": round(floor, 3),
            "vs_launch": round(floor / (per_launch_s * 1e6), 4),
            "how": "torch copy_ (the HIP runtime's device copy) of the same bytes, half each way, over rotated "
                   "buffer pairs (>= 1 GiB), 256 copies timed by events inside one graph",
        },
        "wall_us_per_call_eager": round(t["eager_us"], 2),
        "cpu_baseline": cpu,
        "cpu_oracle": cpu_oracle,
    }
    if info.get("flops"):
        # a matrix-core-bound workload: the roofline is MFMA throughput, the
        # value in TFLOP/s; the HBM rate stays in the record
        tf = info["flops"] / per_launch_s / 1e12
        res["hbm_gbs"] = res["value"]
        res["value"] = round(tf, 2)
        res["unit"] = "TFLOP/s"
        res["pct_of_peak"] = round(100.0 * tf / PEAK_BF16_TFS, 3)
        rf = res["roofline"]
        rf.update({"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFS, "unit": "TFLOP/s",
                   "frac": round(tf / PEAK_BF16_TFS, 5), "flops_per_launch": info["flops"],
                   "achievable": None, "frac_of_achievable": None, "steady_frac": None})
    del launch, info
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


METRIC = "achieved HBM GB/s (% of MI355X peak) + tokens/s for paged KV append/FP8 quant"


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2048)
    p.add_argument("--warmup", type=int, default=256)
    p.add_argument("--workload", default="default",
                   help="default: config 2 as the headline plus every other configuration under `secondary`")
    p.add_argument("--no-secondary", action="store_true", help="default workload: the headline only")
    p.add_argument("--rotate", type=int, default=512, help="rotation sets of inputs/slots")
    p.add_argument("--eager", action="store_true", help="time plain eager launches (host launch rate included)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--detail", default=os.path.join("gpurun_out", "bench_detail.json"),
                   help="file for the full per-workload records ('' for none); the result line stays compact")
    p.add_argument("--transports", default="blit,memcpy", help="swap workload: transports to compare")
    p.add_argument("--swap-reps", type=int, default=3)
    p.add_argument("--num-splits", type=int, default=0, help="decode_attention: splits of the longest sequence (0: auto)")
    p.add_argument("--q-size", type=int, default=-1,
                   help="fp8_prefill_append / bf16_prefill_append: query columns ahead of K and V in each qkv "
                        "row (-1: 4096, Llama-3-8B; 0: contiguous K/V rows)")
    p.add_argument("--tokens", type=int, default=0,
                   help="fp8_prefill_append / bf16_prefill_append: new tokens (0: 32768); mla_*: tokens "
                        "(0: config 4's 4096 prefill / 128 decode)")
    p.add_argument("--slots", default="pages", choices=("pages", "contiguous"),
                   help="*_prefill_append: 'pages' scatters the prompt's pages over the cache (the config); "
                        "'contiguous' writes consecutive slots (the same kernel without the page scatter)")
    p.add_argument("--chunked", action="store_true",
                   help="prefill_attention: the decode reader over 2-token chunks instead of the prefill kernel")
    p.add_argument("--block-size", type=int, default=16,
                   help="chunked_append / gather / *_prefill_append: page size (16 is configs 2 and 3; "
                        "128 is config 3's sensitivity run)")
    args = p.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the KV kernels are rank-local; see the sharding notes). Run with --gpus 1.", flush=True)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit("--steps must be >= 1 and --warmup >= 0")

    import torch

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    name = args.workload
    standalone = {"swap": run_swap, "hbm_copy": run_hbm_copy, "swap_sweep": run_swap_sweep,
                  "attention_shapes": run_attention_shapes, "metadata": run_metadata, "l2_cycle": run_l2_cycle}
    if name in standalone:
        return standalone[name](args, device)
    headline = "fp8_decode_append" if name == "default" else name
    if headline not in SETUPS:
        raise SystemExit(f"unknown workload {name}")

    achievable = measure_device_copy(device)
    progress(f"achievable device copy: {achievable:.1f} GB/s")
    nocpu = args.no_cpu_baseline
    res = measure_workload(args, device, headline, args.steps, args.warmup, achievable,
                           cpu_budget=0 if nocpu else 5.0, port_budget=0 if nocpu else 10.0)
    progress(f"{headline}: {res['roofline']['us_per_launch']} us/launch, {res['value']} GB/s")
    secondary = None
    if name == "default" and not args.no_secondary:
        secondary = {}
        for sname, steps, warmup in SECONDARY:
            t0 = time.perf_counter()
            if sname == "swap":
                r = measure_swap(device, ("blit",), reps=steps)
            elif sname == "metadata":
                r = measure_metadata(device)
            elif sname == "l2_cycle":
                r = measure_l2_cycle(device, steps)
            else:
                r = measure_workload(args, device, sname, steps, warmup, achievable,
                                     cpu_budget=0 if nocpu else 1.0, port_budget=0)
            secondary[sname] = r
            progress(f"{sname}: {r['value']} {r['unit']} ({time.perf_counter() - t0:.1f} s)")
    full = dict(headline=dict(res, name=headline), secondary=secondary, cpu_model=_cpu_model(),
                cpus_visible=os.cpu_count(), args=vars(args))
    detail = write_detail(args.detail, full)
    print(json.dumps(result_line(res, args.warmup, secondary, detail), separators=(",", ":")), flush=True)


def write_detail(path, full):
    """Write the full per-workload records (configs, timings, copy floors, CPU
    baselines) as JSON to `path`; returns the path written, or None."""
    if not path:
        return None
    try:
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "w") as f:
            json.dump(full, f, indent=1)
        return path
    except OSError as e:
        progress(f"could not write {path}: {e}")
        return None


def _short_config(cfg):
    keep = ("workload", "tokens", "valid_tokens", "kv_heads", "head_dim", "block_size", "num_blocks", "cache_dtype",
            "scale", "rotation_sets", "timing")
    return {k: cfg[k] for k in keep if k in cfg}


def _short_cpu(cpu):
    if not cpu:
        return None
    out = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "value_1thread") if k in cpu}
    out["sample"] = cpu.get("sample", "")[:160]
    return out


def result_line(res, warmup, secondary, detail=None):
    """The one JSON result line (a few KB): the headline's fields in full, each
    secondary workload as its value, roofline fraction, per-launch time and
    CPU baseline.  The full records go to the detail file."""
    rf = res["roofline"]
    line = {
        "metric": METRIC,
        "value": res["value"],
        "unit": res.get("unit", "GB/s"),
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": "synthetic (seeded)",
        "tokens_per_s": res["tokens_per_s"],
        "pct_of_peak": res["pct_of_peak"],
        "config": _short_config(res["config"]),
        "roofline": {k: rf[k] for k in ("bound", "kernel", "achieved", "peak", "unit", "frac", "traffic",
                                        "bytes_per_launch", "us_per_launch", "steady_us_per_launch", "steady_frac",
                                        "achievable", "frac_of_achievable") if k in rf},
        "copy_floor_us": None if not res.get("copy_floor") else res["copy_floor"]["us"],
        "cpu_baseline": _short_cpu(res.get("cpu_baseline")),
        "cpu_oracle": _short_cpu(res.get("cpu_oracle")),
    }
    if secondary is not None:
        sec = {}
        for k, r in secondary.items():
            rr = r.get("roofline") or {}
            cpu = r.get("cpu_baseline") or {}
            e = {"value": r["value"], "unit": r["unit"]}
            if rr.get("frac") is not None:
                e["frac"] = rr["frac"]
            if rr.get("us_per_launch") is not None:
                e["us"] = rr["us_per_launch"]
            elif r.get("ms_per_step") is not None:
                e["ms"] = round(r["ms_per_step"], 3)
            if r.get("copy_floor"):
                e["copy_us"] = r["copy_floor"]["us"]
            if cpu:
                e["cpu"] = cpu.get("value")
                if cpu.get("unit") != r["unit"]:
                    e["cpu_unit"] = cpu.get("unit")
                if cpu.get("cores") is not None:
                    e["cpu_cores"] = cpu["cores"]
            sec[k] = e
        line["secondary"] = sec
    if detail:
        line["detail"] = detail
    return line


if __name__ == "__main__":
    main()
