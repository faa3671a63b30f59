"""PyTorch-CPU attention: the CPU path timed beside the GPU (test/bench only).

This is the comparator the reference's own tests call,
``F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0,
is_causal=..., scale=...)`` (``tests/test_correctness.py:43-45, 75-77``),
run on the host in float32 on the same fp16 inputs upcast once.  It is a
second, independent implementation of the oracle's math and the
``cpu_baseline`` leg of ``bench.py``; the shipped path never calls it.
"""

from __future__ import annotations

import numpy as np

from .attention import resolve_sm_scale


def to_cpu_f32(q16, k16, v16):
    """Upcast fp16 numpy arrays to contiguous float32 CPU tensors."""
    import torch

    return tuple(torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
                 for x in (q16, k16, v16))


def sdpa_cpu_f32(q, k, v, sm_scale=0.0, causal=False):
    """``F.scaled_dot_product_attention`` on float32 CPU tensors."""
    import torch.nn.functional as F

    scale = resolve_sm_scale(sm_scale, q.shape[-1])
    return F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0,
                                          is_causal=causal, scale=scale)
