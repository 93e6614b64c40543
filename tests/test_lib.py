"""The C ABI library loads and exports what include/pipeswift_kv.h declares.

CPU-only: argument checks that return before any HIP call are exercised, no
kernel is launched.
"""

import ctypes
import os
import re

import numpy as np
import pytest

from pipeswift_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "pipeswift_kv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(psk_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.EXPORTED_SYMBOLS), "ctypes signatures and header disagree"
    assert lib.psk_abi_version() == 1


def test_argument_errors_return_before_any_device_call():
    lib = _lib.lib()
    z = _lib.i64_array([0, 0, 0, 1])
    st = lib.psk_reshape_and_cache(None, None, None, None, None, 4, 0, 128, 16, 8, 0, 0, z, z, 2, 2,
                                   None, None, None)
    assert st == -1 and b"bad sizes" in lib.psk_last_error()
    st = lib.psk_reshape_and_cache(None, None, None, None, None, 4, 8, 128, 16, 8, 0, 0, z, z, 2, 0,
                                   None, None, None)
    assert st == -2
    # zero tokens is a no-op, even with NULL pointers (impl_utils returns early too)
    assert lib.psk_reshape_and_cache(None, None, None, None, None, 0, 8, 128, 16, 8, 0, 0, z, z, 2, 3,
                                     None, None, None) == 0
    with pytest.raises(AssertionError, match="bad sizes"):
        _lib.check(lib.psk_gather_cache(None, None, None, None, None, None, None, 1, 1, 1, 0, 16, 8, 1, 1, 1,
                                        2, 2, None, None), "gather")
    assert lib.psk_kv_amax_workspace_len() >= 2
    # copy_blocks' grid limits: one workgroup per (pair, layer) on a 2-D grid
    fake = 1 << 20  # never dereferenced: the checks return first
    st = lib.psk_copy_blocks(fake, 70000, 65536, 65536, 65536, 4, fake, 8, None)
    assert st == -1 and b"num_layers 70000 exceeds 65535" in lib.psk_last_error()
    st = lib.psk_copy_blocks(fake, 2, 65536, 65536, 65536, 4, fake, (1 << 24) + 1, None)
    assert st == -1 and b"exceeds 2^24" in lib.psk_last_error()
    st = lib.psk_copy_blocks(fake, 2, 65536, 1024, 65536, 4, fake, 8, None)
    assert st == -1 and b"exceeds block_stride" in lib.psk_last_error()
    assert lib.psk_copy_blocks(None, 2, 65536, 65536, 65536, 4, None, 0, None) == 0  # no pairs: no-op


def test_mla_fp8_tile_sizes_and_dtypes_are_checked_on_the_host():
    lib = _lib.lib()
    assert lib.psk_mla_fp8_tile_entry_bytes(512, 64) == 656
    assert lib.psk_mla_fp8_tile_entry_bytes(100, 64) == -1
    assert lib.psk_mla_fp8_tile_entry_bytes(512, 3) == -1
    assert lib.psk_mla_fp8_tile_entry_bytes(128 * 65, 0) == -1
    st = lib.psk_concat_and_cache_mla_fp8_tiles(None, None, None, None, 4, 512, 64, 512, 64, 64, 10, 64 * 656, 656,
                                                1, None)  # fp16 input
    assert st == -2 and b"bf16" in lib.psk_last_error()
    st = lib.psk_concat_and_cache_mla_fp8_tiles(None, None, None, None, 4, 512, 64, 512, 64, 64, 10, 64 * 600, 600,
                                                2, None)  # entry longer than the page stride
    assert st == -1 and b"656-byte entry" in lib.psk_last_error()
    assert lib.psk_concat_and_cache_mla_fp8_tiles(None, None, None, None, 0, 512, 64, 512, 64, 64, 10, 64 * 656,
                                                  656, 2, None) == 0
    st = lib.psk_gather_mla_fp8_tiles(None, None, None, None, None, 1, 4, 8, 512, 64, 64, 10, 64 * 656, 656,
                                      576 * 2, 1, None)  # fp16 output
    assert st == -2


def test_swap_range_is_checked_on_the_host():
    lib = _lib.lib()
    u = (ctypes.c_uint64 * 1)(0)
    b = (ctypes.c_uint64 * 1)(4096)
    s = _lib.i64_array([5])
    d = _lib.i64_array([0])
    n = _lib.i64_array([2])
    st = lib.psk_swap_blocks(_lib.SWAP_MEMCPY, u, u, b, 1, s, d, n, 1, 6, 10, None, 0, None, 0, None)
    assert st == -3 and b"src pages [5, 7)" in lib.psk_last_error()
    st = lib.psk_swap_blocks(_lib.SWAP_BLIT, u, u, b, 1, d, d, n, 1, 6, 10, None, 0, None, 0, None)
    assert st == -4
    assert lib.psk_swap_staging_bytes(2, 10) >= 2 * 24 + 2 * 10 * 8


def test_build_flags_disable_packed_fp32():
    import __graft_entry__ as g

    flags = " ".join(g.FLAGS)
    assert "-packed-fp32-ops" in flags and "gfx950" in flags
