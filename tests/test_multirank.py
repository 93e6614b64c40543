"""Cross-rank agreement over a gloo process group (CPU, world size 2): the
page ledger's minimum over ranks (BlockManager._min_across_workers, the
all-reduce MIN of the reference's mpu.py:31-47) and the L2 page count every
rank agrees on (_L2Tier._agreed_num_pages, block_manager.py:233-267)."""

import multiprocessing as mproc
import os
import socket
import warnings


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _rank(rank, world, port, out):
    import torch
    import torch.distributed as dist

    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        from pipeswift_amd.block_manager import BlockManager, _L2Tier

        low = BlockManager._min_across_workers(100 - 30 * rank)
        # [layers, pages, 2, page_size, heads, head_dim] bf16: 16 KiB per page
        caches = [torch.zeros(2, 8, 2, 16, 2, 64, dtype=torch.bfloat16)]
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            # rank r budgets (r + 1) x 64 KiB of host memory: 4 or 8 pages
            pages = _L2Tier._agreed_num_pages(8, (rank + 1) * 64 / 1024**2, caches, BlockManager._min_across_workers)
        out.put((rank, low, pages, [str(w.message) for w in caught]))
    finally:
        dist.destroy_process_group()


def test_ledger_sizes_agree_over_two_gloo_ranks():
    ctx = mproc.get_context("spawn")
    out = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_rank, args=(r, 2, port, out)) for r in range(2)]
    for p in procs:
        p.start()
    try:
        res = sorted(out.get(timeout=180) for _ in procs)
    finally:
        for p in procs:
            p.join(timeout=60)
    assert [p.exitcode for p in procs] == [0, 0]
    for rank, low, pages, msgs in res:
        assert low == 70, (rank, low)
        assert pages == 4, (rank, pages)
        assert any("fewer pages than the GPU pool" in m for m in msgs), msgs
        assert any("lowered to the minimum" in m for m in msgs) == (rank == 1), msgs
