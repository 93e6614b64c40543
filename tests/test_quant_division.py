"""The FP8 quantizer, proven on the CPU against the IEEE quotient path.

The append kernels quantize in sign-magnitude form without a per-element
division: r = RN(1/s) once per wave, y = RN(|x|*r), e = fma(-y, s, |x|),
m = fma(e, r, y), byte = e4m3(min(m, 448)) | sign(x), inside a
[2^-80, 2^100) gate on |s| (pipeswift_amd/csrc/psk_common.h), with a NaN
quotient stored by policy (0xFE, the reference append's Triton clamp, or
0x7F|sign, torch's).  The reference divides in fp32 (fp8_kv.py:75-77,
reshape_and_cache.py:66-77).  oracle/quant_check.c restates the kernel
sequence in host IEEE binary32 arithmetic (the kernels run with f32 denormals
preserved) and sweeps, under both NaN policies:

  * every bf16 input pattern against the scale RN(a/448) of every finite
    positive bf16 amax a (2.1e9 cases: every per-tensor scale the amax kernel
    can produce for a bf16 tensor), and the same for f16;
  * sampled fp32 inputs and scales, including an adversarial set whose
    quotients lie just below a power of two, where RN(x * RN(1/s)) can miss
    x/s by more than an ulp, and scales a few ulps either side of the gate.

Result: the clamped magnitude the kernel converts equals |clamp(x/s)| bit for
bit whenever that is >= 2^-20, and every E4M3 byte is the same everywhere
(below 2^-20 both round to a zero of the input's sign).  Planted mistakes (the
correction step or the gate removed) are detected by the same sweeps.  The
host E4M3 conversion is pinned against torch's CPU float8_e4m3fn conversion,
and the host kernel sequence against torch's (x / s).clamp().to(e4m3).
"""

import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "libquant_check.so")
GOLDEN = os.path.join(ROOT, "tests", "golden", "e4m3_of_bf16.bin")

BF16, F16 = 0, 1
KERNEL, NO_CORRECTION, NO_GATE = 0, 1, 2
N_FINITE_POS = {BF16: 0x7F80 - 1, F16: 0x7C00 - 1}


@pytest.fixture(scope="module")
def qc():
    if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(LIB.replace("libquant_check.so",
                                                                                        "quant_check.c")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(LIB)
    p = ctypes.c_void_p
    lib.qc_e4m3.argtypes = [p, ctypes.c_int64, p]
    lib.qc_quantize.argtypes = [p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, p]  # policy: 0 clamp_min, 1 torch
    lib.qc_sweep_all.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, p, p]
    lib.qc_sweep_random.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, p, p]
    return lib


FIELDS = ("cases", "fast", "mag_bad", "byte_bad", "big_bad")
CLAMP_MIN, TORCH = 0, 1


def _sweep_all(qc, kind, variant=KERNEL):
    out = np.zeros(5, np.int64)
    bad = np.zeros(3, np.uint32)
    qc.qc_sweep_all(kind, kind, variant, out.ctypes.data, bad.ctypes.data)
    return dict(zip(FIELDS, out.tolist())), bad


def _sweep_random(qc, mode, n, variant=KERNEL, seed=20260101):
    out = np.zeros(5, np.int64)
    bad = np.zeros(3, np.uint32)
    qc.qc_sweep_random(seed, n, mode, variant, out.ctypes.data, bad.ctypes.data)
    return dict(zip(FIELDS, out.tolist())), bad


def test_host_e4m3_conversion_matches_torch(qc):
    """The checker's clamp + E4M3FN conversion equals torch's on every bf16
    pattern (the committed golden table) and on 2^20 random fp32 values
    spread over the E4M3 range, its subnormals and beyond."""
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float().numpy()
    out = np.empty(65536, np.uint8)
    qc.qc_e4m3(x.ctypes.data, 65536, out.ctypes.data)
    assert np.array_equal(out, np.fromfile(GOLDEN, np.uint8))

    g = torch.Generator().manual_seed(11)
    mag = torch.exp2(torch.empty(1 << 20).uniform_(-14.0, 10.0, generator=g))
    sign = torch.where(torch.rand(1 << 20, generator=g) < 0.5, -1.0, 1.0)
    xf = (mag * sign).float()
    want = xf.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    xn = xf.numpy()
    got = np.empty(xn.shape[0], np.uint8)
    qc.qc_e4m3(xn.ctypes.data, xn.shape[0], got.ctypes.data)
    assert np.array_equal(got, want)


def test_host_kernel_sequence_matches_torch_division_on_golden_set(qc):
    """qc_quantize (the kernel's sequence) against torch's (x / s).clamp().to(e4m3)
    on the committed golden set of ties, subnormals and saturation edges, and
    on every bf16 pattern at scale 1 (the golden table, torch NaN policy)."""
    z = np.load(os.path.join(ROOT, "tests", "golden", "e4m3_scaled.npz"))
    x, s, q = z["x"], z["scale"], z["q"]
    for sv in np.unique(s):
        m = s == sv
        xs = np.ascontiguousarray(x[m])
        got = np.empty(xs.shape[0], np.uint8)
        qc.qc_quantize(xs.ctypes.data, xs.shape[0], float(sv), TORCH, got.ctypes.data)
        assert np.array_equal(got, q[m]), f"scale {sv}"
    xb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float().numpy()
    got = np.empty(65536, np.uint8)
    qc.qc_quantize(xb.ctypes.data, 65536, 1.0, TORCH, got.ctypes.data)
    golden = np.fromfile(GOLDEN, np.uint8)
    assert np.array_equal(got, golden)
    qc.qc_quantize(xb.ctypes.data, 65536, 1.0, CLAMP_MIN, got.ctypes.data)
    nan = np.isnan(xb)
    assert np.array_equal(got[~nan], golden[~nan]) and (got[nan] == 0xFE).all()


@pytest.mark.parametrize("kind", [BF16, F16], ids=["bf16", "f16"])
def test_division_exact_for_every_16bit_input_and_every_amax_scale(qc, kind):
    r, bad = _sweep_all(qc, kind)
    assert r["cases"] == 65536 * N_FINITE_POS[kind]
    assert r["byte_bad"] == 0, f"E4M3 byte differs, first case x={bad[0]:#x} s={bad[1]:#x} got={bad[2]:#x}"
    assert r["big_bad"] == 0, f"magnitude >= 2^-20 differs, first case x={bad[0]:#x} s={bad[1]:#x}"
    if kind == F16:
        # every f16 amax gives a scale inside the gate, and every f16 magnitude is exact
        assert r["fast"] == r["cases"] and r["mag_bad"] == 0


@pytest.mark.parametrize("mode", [0, 1, 2, 3], ids=["random", "near_binade_top", "mid_range", "gate_edges"])
def test_division_exact_on_sampled_fp32(qc, mode):
    r, bad = _sweep_random(qc, mode, 50_000_000)
    assert r["cases"] == 50_000_000
    assert r["byte_bad"] == 0 and r["big_bad"] == 0, f"x={bad[0]:#x} s={bad[1]:#x} got={bad[2]:#x}"
    if mode in (1, 2):
        assert r["fast"] == r["cases"] and r["mag_bad"] == 0


def test_sweeps_detect_planted_mistakes(qc):
    """The same sweeps fail for plausible wrong kernels: without the FMA
    correction (quotient RN(x * RN(1/s))) bytes differ, and without the range
    gate the tiny-scale cases break."""
    r, _ = _sweep_all(qc, BF16, NO_CORRECTION)
    assert r["byte_bad"] > 0 and r["big_bad"] > 0
    r, _ = _sweep_random(qc, 1, 5_000_000, NO_CORRECTION)
    assert r["big_bad"] > 0
    r, _ = _sweep_all(qc, BF16, NO_GATE)
    assert r["big_bad"] > 0
