"""CPU oracle for the FlashAttention-2 forward path.

Test infrastructure only: ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or the timed CPU comparator).  The product path in ``flashlite_amd``
never imports it.

The reference's own implementation (CUDA C++ with ``nvcuda::wmma`` and inline
PTX) cannot be compiled in this image -- no nvcc, no CUDA headers -- so there
is no ``oracle/_ref`` build; the restatement is pinned by closed forms,
brute force, torch-CPU SDPA and committed fixtures instead.
"""

from .attention import (  # noqa: F401
    LOG2_E,
    attention_bruteforce,
    attention_bytes,
    attention_flops,
    attention_fp32,
    attention_fp64,
    attention_lse,
    causal_visible,
    error_stats,
    resolve_sm_scale,
    sm_scale_log2,
)
