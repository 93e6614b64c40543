"""CPU oracle for the paged KV-cache data path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference (wsjdsg/PipeSwift) computes
on the KV-cache write/read/copy path, so the HIP kernels can be checked against
it byte for byte.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or as
the timed CPU baseline: the product package ``pipeswift_amd`` never imports it
and has no CPU fallback.

Each function cites the reference lines it follows.  How each one is pinned
(beyond restating the reference) is recorded in its docstring; the pins
themselves live in ``tests/test_oracle.py``:

* ``e4m3fn_from_f32`` / ``e4m3fn_to_f32`` / ``bf16_from_f32``: exhaustive
  comparison with torch's CPU dtype conversions (library routines) over every
  bf16 and fp8 bit pattern, plus the committed golden table
  ``tests/golden/e4m3_of_bf16.bin``.
* append / MLA concat / gather / copy_blocks: torch ``index_put_`` /
  ``index_select`` on the same strided layout, literal hand-computed tiny
  cases, untouched-slot sentinels and the round trip gather(append(x)) == x.
* coalesce / range check / slot mapping: brute force on small random inputs.
"""
