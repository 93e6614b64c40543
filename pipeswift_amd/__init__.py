"""MI355X-native paged KV-cache data path for PipeSwift.

Hand-written gfx950 HIP kernels behind a C ABI (include/pipeswift_kv.h,
libpipeswift_kv.so), with the reference's Python cache API on top:

  reshape_and_cache   reshape_and_cache_flash / _diffkv (+ the triton_* names)
  impl_utils          append_kv_cache / append_mla_kv_cache
  metadata            KVCacheInfo, prepare_kv_info (slot_mapping, page_table)
  cudagraph           static metadata for graph replay
  cache_ops           gather_cache, copy_blocks, compute_kv_scales
  copy_engine         CopyEngine / CopyHandle (DRAM L2 offload, swap_blocks)
  fp8_kv              FP8 constants, flag and scale helpers
"""

from .cache_ops import compute_kv_scales, copy_blocks, gather_cache
from .impl_utils import append_kv_cache, append_mla_kv_cache
from .metadata import KVCacheInfo, prepare_kv_info
from .reshape_and_cache import (
    reshape_and_cache_flash,
    reshape_and_cache_flash_diffkv,
    triton_reshape_and_cache_flash,
    triton_reshape_and_cache_flash_diffkv,
)

__all__ = [
    "KVCacheInfo",
    "append_kv_cache",
    "append_mla_kv_cache",
    "compute_kv_scales",
    "copy_blocks",
    "gather_cache",
    "prepare_kv_info",
    "reshape_and_cache_flash",
    "reshape_and_cache_flash_diffkv",
    "triton_reshape_and_cache_flash",
    "triton_reshape_and_cache_flash_diffkv",
]
