"""ctypes binding of libpipeswift_kv.so, the gfx950 C ABI of the KV-cache path.

The library is built in-tree (``__graft_entry__.build()`` or
``make -C pipeswift_amd/csrc``) next to this file.  There is no fallback: if the
library is missing every operation raises, so nothing can silently run a
non-HIP path.  Status codes follow include/pipeswift_kv.h: negative values are
precondition failures (AssertionError, matching the reference's Python
asserts), positive values are hipError_t (RuntimeError, matching the
reference's driver-failure path, copy_engine.py:454-457).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpipeswift_kv.so")

DTYPE_CODES = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float8_e4m3fn: 3,
}

SWAP_MEMCPY = 0
SWAP_BLIT = 2

_c_int64_p = ctypes.POINTER(ctypes.c_int64)
_c_uint64_p = ctypes.POINTER(ctypes.c_uint64)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> (restype, argtypes)
_SIGNATURES = {
    "psk_last_error": (ctypes.c_char_p, []),
    "psk_abi_version": (_int, []),
    "psk_reshape_and_cache": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_int64_p, _c_int64_p, _int, _int,
         _vp, _vp, _vp],
    ),
    "psk_concat_and_cache_mla": (
        _int,
        [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _vp, _vp],
    ),
    "psk_gather_cache": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int,
         _vp, _vp],
    ),
    "psk_copy_blocks": (_int, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "psk_swap_blocks": (
        _int,
        [_int, _c_uint64_p, _c_uint64_p, _c_uint64_p, _i64, _c_int64_p, _c_int64_p, _c_int64_p, _i64, _i64, _i64,
         _vp, _i64, _vp, _i64, _vp],
    ),
    "psk_swap_staging_bytes": (_i64, [_i64, _i64]),
    "psk_coalesce_runs": (_i64, [_c_int64_p, _c_int64_p, _i64, _c_int64_p, _c_int64_p, _c_int64_p]),
    "psk_kv_amax_scale": (
        _int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _int, ctypes.c_float, _vp, _vp, _vp, _i64, _vp],
    ),
    "psk_kv_amax_workspace_len": (_i64, []),
    "psk_reshape_and_cache_amax": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_int64_p, _c_int64_p, _int,
         ctypes.c_float, _vp, _vp, _vp, _i64, _vp],
    ),
    "psk_kv_amax_scale_noalloc": (
        _int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _int, ctypes.c_float, _vp, _vp, _vp],
    ),
    "psk_build_kv_metadata": (
        _i64,
        [_i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _i64, _vp, _vp, _vp, _vp, _vp, _i64],
    ),
    "psk_refresh_graph_metadata": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64,
         ctypes.c_int32, _vp],
    ),
    "psk_build_next_decode_metadata": (
        _i64, [_i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp],
    ),
    "psk_host_alloc": (_int, [_i64, ctypes.POINTER(ctypes.c_void_p)]),
    "psk_host_free": (_int, [_vp]),
    "psk_keyed_hash": (_int, [_vp, _i64, ctypes.c_uint64, _int, _vp]),
    "psk_page_hash_chain": (_i64, [_vp, _i64, _i64, _i64, ctypes.c_uint64, _int, _vp, _i64]),
    "psk_paged_decode_attention": (
        _int,
        [_vp, _i64, _i64, _int, _vp, _vp, _c_int64_p, _c_int64_p, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _vp, _int, ctypes.c_float, _vp, _vp, _vp, _c_int64_p, _vp, _i64, _i64, _int, _vp,
         _i64, _vp, _i64, _vp],
    ),
    "psk_paged_decode_workspace_len": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "psk_paged_prefill_attention": (
        _int,
        [_vp, _i64, _i64, _int, _vp, _vp, _c_int64_p, _c_int64_p, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _int, ctypes.c_float, _vp, _vp, _vp, _c_int64_p, _vp, _i64, _i64, _int, _vp, _i64,
         _vp, _i64, _vp],
    ),
    "psk_paged_prefill_workspace_len": (_i64, [_i64]),
    "psk_mla_fp8_tile_entry_bytes": (_i64, [_i64, _i64]),
    "psk_concat_and_cache_mla_fp8_tiles": (
        _int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp],
    ),
    "psk_gather_mla_fp8_tiles": (
        _int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the library once; raise ImportError with the build command if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "from the repository root (hipcc --offload-arch=gfx950)"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = lib().psk_last_error().decode(errors="replace")
    if status < 0:
        raise AssertionError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise AssertionError(f"unsupported dtype {dtype}") from None


# torch's raw accessor of the current stream (what its generated kernels call):
# 0.05 us against 1.7 us for torch.cuda.current_stream(device).cuda_stream, which
# builds a Stream object per call.  The public call is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


_I64x4 = ctypes.c_int64 * 4


def i64_array(values) -> ctypes.Array:
    if len(values) == 4:
        return _I64x4(*values)
    return (ctypes.c_int64 * len(values))(*values)


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
