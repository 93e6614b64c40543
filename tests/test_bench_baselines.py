"""The bench's torch CPU baselines (the reference's host path: index_put_ and
index_select) must compute what the oracle computes, or their GB/s would time
different work.  CPU only."""

import numpy as np
import torch

import bench
from oracle import kv_oracle as O
import workloads


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_torch_append_baseline_matches_oracle_bf16():
    case = workloads.config1_append(seed=5, num_tokens=200, num_blocks=64)
    step, cache = bench.torch_cpu_append_step(case, fp8=False)
    step()
    exp = np.zeros(tuple(case.cache.shape), np.uint16)
    O.reshape_and_cache(_u16(case.key()), _u16(case.value()), exp[:, 0], exp[:, 1], case.slot_mapping.numpy())
    assert np.array_equal(_u16(cache), exp)


def test_torch_append_baseline_matches_oracle_fp8():
    case = workloads.config2_fp8_decode(batch=32, num_blocks=4096, ctx_hi=2048)
    step, cache = bench.torch_cpu_append_step(case, fp8=True)
    step()
    key, value = _u16(case.key()), _u16(case.value())
    ks, _ = O.amax_scale(key, "bf16")
    vs, _ = O.amax_scale(value, "bf16")
    exp = np.zeros(tuple(case.cache.shape), np.uint8)
    O.reshape_and_cache(key, value, exp[:, 0], exp[:, 1], case.slot_mapping.numpy(), "bf16", "fp8", ks, vs)
    assert np.array_equal(cache.view(torch.uint8).numpy(), exp)


def test_torch_gather_baseline_matches_oracle():
    cc = workloads.config3_chunked(max_prefix=2000, num_blocks=2048)
    step, out = bench.torch_cpu_gather_step(cc)
    step()
    bt, cu = cc.block_table.numpy(), cc.cu_seq_lens.numpy()
    assert np.array_equal(_u16(out[0]), O.gather_cache(_u16(cc.append.cache[:, 0]), bt, cu))
    assert np.array_equal(_u16(out[1]), O.gather_cache(_u16(cc.append.cache[:, 1]), bt, cu))


def test_timed_launch_count_is_exactly_the_requested_steps():
    """The bench captures exactly --steps launches (the driver runs --steps 20;
    an earlier version replayed only whole 64-launch graphs and timed none)."""
    for rotate in (1, 4, 8, 512):
        for steps in (1, 5, 20, 63, 64, 65, 127, 2048):
            sets = bench.launch_sets(steps, rotate)
            assert len(sets) == steps
            assert sets == [i % rotate for i in range(steps)]
    assert bench.launch_sets(0, 8) == []


def test_torch_mla_baseline_matches_oracle():
    case = workloads.config4_mla(num_tokens=64, num_blocks=100, decode=True)
    step, cache = bench.torch_cpu_mla_step(case, None)
    step()
    exp = np.zeros(tuple(case.cache.shape), np.uint16)
    O.concat_and_cache_mla(_u16(case.kv_c), _u16(case.k_pe()), exp, case.slot_mapping.numpy())
    assert np.array_equal(_u16(cache), exp)


def test_torch_decode_attention_baseline_matches_oracle():
    """The torch host attention that the decode-attention workloads report as
    their CPU baseline computes what the float64 oracle computes (queries
    already on the E4M3 grid, so the oracle's query quantization is exact)."""
    g = torch.Generator().manual_seed(11)
    P, ps, H, D, Hq, B = 64, 16, 2, 64, 8, 3
    kc = (torch.randn(P, ps, H, D, generator=g) * 2).to(torch.float8_e4m3fn)
    vc = (torch.randn(P, ps, H, D, generator=g) * 2).to(torch.float8_e4m3fn)
    ctx = torch.tensor([37, 16, 90])
    bt = torch.stack([torch.randperm(P, generator=g)[:8] for _ in range(B)]).to(torch.int32)
    scales = torch.tensor([0.5, 0.25])
    for q_len in (1, 4):
        q = (torch.randn(B * q_len, Hq, D, generator=g)).to(torch.float8_e4m3fn).to(torch.bfloat16)
        step, outs, nbytes = bench.torch_cpu_decode_attention_step(kc, vc, bt, ctx, q, scales, q_len)
        step()
        assert nbytes > 0
        exp, _ = O.paged_decode_attention(
            _u16(q), "bf16", kc.view(torch.uint8).numpy(), vc.view(torch.uint8).numpy(), bt.numpy(),
            ctx.numpy(), D ** -0.5, None, np.full((B, H), 0.5, np.float32), np.full((B, H), 0.25, np.float32),
            cu_seqlens_q=np.arange(B + 1) * q_len, causal=True)
        got = torch.cat(outs).double().numpy()
        np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-5)


def _stub_record(name, us=2.0):
    return {"value": 123.45, "unit": "GB/s", "steps": 20, "warmup": 5, "ms_per_step": us / 1e3,
            "tokens_per_s": 1e8, "pct_of_peak": 1.5, "dtype": "fp8_e4m3fn",
            "config": {"workload": name + " " + "x" * 400, "tokens": 128, "timing": "t" * 300, "extra": "y" * 2000},
            "roofline": {"bound": "hbm", "kernel": "k" * 60, "achieved": 123.45, "peak": 8000.0, "unit": "GB/s",
                         "frac": 0.01543, "traffic": 827707, "bytes_per_launch": 787456, "us_per_launch": us,
                         "steady_us_per_launch": us, "steady_frac": 0.02, "achievable": 6100.0,
                         "frac_of_achievable": 0.02},
            "copy_floor": {"us": 2.2, "vs_launch": 1.1, "how": "h" * 300},
            "cpu_baseline": {"value": 7.9, "unit": "GB/s", "cores": 16, "kind": "port", "value_1thread": 1.0,
                             "sample": "s" * 500},
            "cpu_oracle": {"value": 0.6, "unit": "GB/s", "cores": 1, "kind": "port", "sample": "o" * 500}}


def test_result_line_is_one_compact_json_line_with_every_baseline():
    """The driver reads the last line of the run's output, from a tail of a
    few KB: the result line must stay one short JSON line even with every
    secondary workload present, and carry roofline and CPU baselines."""
    import json

    secondary = {name: _stub_record(name) for name, _, _ in bench.SECONDARY}
    secondary["swap"]["roofline"]["us_per_launch"] = None
    line = bench.result_line(_stub_record("fp8_decode_append"), 5, secondary, "gpurun_out/bench_detail.json")
    text = json.dumps(line, separators=(",", ":"))
    assert "\n" not in text
    assert len(text) < 4096, len(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in line["roofline"], key
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in line["cpu_baseline"], key
    assert set(line["secondary"]) == {name for name, _, _ in bench.SECONDARY}
    assert all(e.get("cpu") is not None for e in line["secondary"].values())


def test_bench_prints_no_json_and_nothing_to_stderr_besides_the_result():
    """Progress lines are plain text on stdout; the source has no stderr
    prints, so the result line is the last line of the combined output."""
    import inspect
    import io
    import contextlib

    src = inspect.getsource(bench)
    assert "sys.stderr" not in src.replace("nothing goes to stderr", "")
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        bench.progress("x: 1.0 GB/s")
    assert not buf.getvalue().lstrip().startswith("{")
