"""FP8 (OCP E4M3FN) KV-cache settings.

Mirrors pipeswift/utils/fp8_kv.py: the dtype and saturation constants
(:24-25), the global flag (:35-41), the attention-reader loader
``attn_varlen_func`` (:44-62), ``check_available`` (:64-71), ``quantize`` (:75-77), the graph-safe warmup
(:80-91) and ``unit_descale`` (:94-103).  The loader hands back this
package's reader (``attention.flash_attn_varlen_func``) in place of vLLM's FA3
fork, so the reference's ``_fp8_paged_attn`` (attention.py:148-187) runs on it
unchanged.

gfx950 converts to the OCP E4M3FN format natively (max 448, 0x7F/0xFF NaN);
this is not MI300's FNUZ variant (max 240).
"""

from __future__ import annotations

import torch

from . import cache_ops

FP8_KV_DTYPE = torch.float8_e4m3fn
FP8_E4M3_MAX = 448.0

_ENABLED = False
_scale_one: dict = {}


def set_enabled(enabled: bool) -> None:
    global _ENABLED
    _ENABLED = bool(enabled)


def is_enabled() -> bool:
    return _ENABLED


def quantize(x: torch.Tensor) -> torch.Tensor:
    """Per-tensor e4m3 cast at scale 1.0, saturating (fp8_kv.py:75-77).

    Elementwise torch on the tensor's device; the cache write itself fuses
    the same conversion into the append kernel.
    """
    return x.clamp(-FP8_E4M3_MAX, FP8_E4M3_MAX).to(FP8_KV_DTYPE)


def warmup(device) -> None:
    """Allocate the unit scale and the amax workspace outside graph capture."""
    assert not torch.cuda.is_current_stream_capturing(), "fp8_kv.warmup must run outside graph capture"
    device = torch.device(device)
    if device not in _scale_one:
        _scale_one[device] = torch.ones((1,), dtype=torch.float32, device=device)
    cache_ops.warmup(device)


def check_available() -> None:
    """Fail at startup rather than in the first forward pass (fp8_kv.py:64-71):
    the FP8 reader and append need a gfx950 GPU and this package's library.

    The reader covers decode, speculative decode and prefill: steps of at
    most 16 query rows per kv head (query tokens x G query heads per kv head)
    run the decode kernels, larger ones the prefill kernel, for groups of up
    to 256 query heads per kv head."""
    assert torch.cuda.is_available(), "--enable_fp8_kv needs a GPU"
    arch = getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", "")
    assert arch.startswith("gfx950"), f"--enable_fp8_kv on this build needs gfx950 (MI355X), got {arch or 'unknown'}"
    from ._lib import lib

    lib()
    attn_varlen_func()


def attn_varlen_func():
    """The FA3-style varlen entry point for the FP8 cache (fp8_kv.py:44-62):
    this package's paged reader, same keywords, for decode, speculative
    decode and prefill."""
    from .attention import flash_attn_varlen_func

    return flash_attn_varlen_func


def unit_descale(num_seqs: int, num_kv_heads: int, device) -> torch.Tensor:
    """``{q,k,v}_descale`` of 1.0 shaped (num_seqs, num_kv_heads) as a
    stride-0 view of one element: no allocation per call, graph safe
    (fp8_kv.py:94-103)."""
    return unit_scale(device).expand(num_seqs, num_kv_heads)


def unit_scale(device) -> torch.Tensor:
    """A one-element fp32 1.0 on ``device`` (the reference's fixed scale)."""
    device = torch.device(device)
    if device not in _scale_one:
        warmup(device)
    return _scale_one[device]
