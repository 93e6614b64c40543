"""psk_kv_amax_scale_noalloc (scratch inside the library, no workspace) against
psk_kv_amax_scale (caller's workspace), both called through the C ABI: the
scales and amax values must be bit-identical, on two calls in a row where the
second has a smaller input, for strided bf16 K/V views, a single contiguous
tensor and fp32/f16 inputs; and against the oracle's amax / 448."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from pipeswift_amd._lib import DTYPE_CODES, lib

pytestmark = pytest.mark.gpu


def _raw16(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _call_pair(k, v, dev):
    """(scales, amax) from the workspace entry and from the no-alloc entry."""
    rows = k.shape[0]
    row_len = k[0].numel()
    s0 = k.stride(0)
    s1 = v.stride(0) if v is not None else s0
    code = DTYPE_CODES[k.dtype]
    stream = torch.cuda.current_stream(dev).cuda_stream
    n = 2 if v is not None else 1
    ws = torch.empty(int(lib().psk_kv_amax_workspace_len()), dtype=torch.int32, device=dev)
    outs = []
    for which in ("workspace", "noalloc"):
        sc = torch.full((n,), -7.0, dtype=torch.float32, device=dev)
        am = torch.full((n,), -7.0, dtype=torch.float32, device=dev)
        vp = None if v is None else v.data_ptr()
        if which == "workspace":
            st = lib().psk_kv_amax_scale(k.data_ptr(), vp, rows, row_len, s0, s1, code, ctypes.c_float(448.0),
                                         sc.data_ptr(), am.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        else:
            st = lib().psk_kv_amax_scale_noalloc(k.data_ptr(), vp, rows, row_len, s0, s1, code,
                                                 ctypes.c_float(448.0), sc.data_ptr(), am.data_ptr(), stream)
        assert st == 0, lib().psk_last_error().decode()
        torch.cuda.synchronize()
        outs.append((sc.cpu().view(torch.int32).numpy().copy(), am.cpu().view(torch.int32).numpy().copy()))
    return outs


def test_noalloc_amax_matches_workspace_entry_bf16_kv_views(dev):
    g = torch.Generator().manual_seed(2024)
    for tokens in (128, 16):  # second call smaller: the scratch keeps the first call's partials
        qkv = (torch.randn(tokens, 6144, generator=g) * 2.0)
        mask = torch.rand(tokens, 6144, generator=g) < 0.01
        qkv = torch.where(mask, qkv * 20.0, qkv).to(torch.bfloat16).to(dev)
        k = qkv[:, 4096:5120].view(tokens, 8, 128)
        v = qkv[:, 5120:6144].view(tokens, 8, 128)
        (ws_s, ws_a), (na_s, na_a) = _call_pair(k, v, dev)
        assert np.array_equal(ws_s, na_s) and np.array_equal(ws_a, na_a), f"{tokens} tokens"
        for j, t in enumerate((k, v)):
            s, a = O.amax_scale(_raw16(t), "bf16")
            assert na_s.view(np.float32)[j] == np.float32(s) and na_a.view(np.float32)[j] == np.float32(a)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
def test_noalloc_amax_matches_workspace_entry_single_tensor(dev, dtype):
    g = torch.Generator().manual_seed(7)
    for n in (1 << 20, 1000):  # a million elements, then a small odd size
        x = (torch.randn(n, generator=g) * 3.0).to(dtype).to(dev).view(n, 1)
        (ws_s, ws_a), (na_s, na_a) = _call_pair(x, None, dev)
        assert np.array_equal(ws_s, na_s) and np.array_equal(ws_a, na_a), f"{n} elements"
        amax = float(x.float().abs().max())
        assert na_a.view(np.float32)[0] == np.float32(amax)
