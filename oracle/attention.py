"""CPU oracle for the FlashAttention-2 forward path (test infrastructure only).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path is the HIP library under ``flashlite_amd/``; it
never routes through anything here.

What it restates (reference = thebigblender/FlashLite, files under
``/root/reference``):

* ``attention_fp32`` / ``attention_fp64`` -- the math every reference kernel
  computes, ``O = softmax(Q.K^T * sm_scale + M) . V`` per (batch, head), with
  ``M`` the top-left aligned causal mask (key ``j`` visible to query ``i`` iff
  ``j <= i``).  Mask semantics follow ``csrc/kernel_flash2.cu:180-230`` (Br=64
  kernel) and ``:521-571`` (Br=128 kernel); the naive kernel's
  ``csrc/kernel_naive.cu:176-214``.  Masked logits are dropped exactly (the
  reference writes -1e30 and then zeroes their probability,
  ``kernel_flash2.cu:299-309``), so a row's weights are a softmax over its
  visible keys only.  Every row has at least one visible key when
  ``N_q == N_k`` (key 0), so no row is fully masked.
* N_k != N_q (not supported by the reference, which indexes K and V with
  N_q, ``kernel_flash2.cu:84, :425``): keys are K's own rows, and the causal
  diagonal is aligned bottom-right -- key ``j`` visible to query ``i`` iff
  ``j <= i + N_k - N_q`` (the convention of PyTorch's ``causal_lower_right``
  and of the ``flash_attn`` package).  A query row with no visible key
  returns 0, which is the reference's fully-masked-row rule
  (``inv_l = l > 0 ? 1/l : 0``, ``kernel_flash2.cu:364-365``).
* ``attention_lse`` -- each row's log-sum-exp ``ln sum_j exp(s_ij)`` over
  its visible keys (``-inf`` for a row with none): the quantity a flash
  kernel's (m, l) state encodes, ``m * ln 2 + ln l`` in the reference's
  base-2 units (``kernel_flash2.cu:251-254, :339``); the reference itself
  does not return it.
* ``resolve_sm_scale`` -- the ``sm_scale == 0.0`` sentinel meaning
  ``1/sqrt(D)`` computed in float32 (``kernel_flash2.cu:769-771``,
  ``kernel_naive.cu:278-280``) and the base-2 prescale
  ``float(sm_scale * log2(e))`` (``kernel_flash2.cu:772``).
* ``attention_flops`` / ``attention_bytes`` -- the benchmark's work formulas
  (``benchmarks/benchmark_throughput.py:23-31``): ``4.B.H.N^2.D`` flops,
  halved for causal; bytes = Q, K, V read once and O written once.

Pins (see ``tests/test_oracle.py``): brute-force scalar loops in float64 on
tiny shapes, torch-CPU ``scaled_dot_product_attention`` (the comparator the
reference's own tests use, ``tests/test_correctness.py:43-45, 75-77``),
closed forms (causal row 0 equals V[0]; constant keys give the (prefix) mean
of V; one-hot peaked scores select a single V row), invariances (score
shift, joint key/value permutation when non-causal, causal independence of
later keys), and the committed C0 golden fixture.
"""

from __future__ import annotations

import math

import numpy as np

LOG2_E = 1.4426950408889634  # log2(e), the mathematical constant


def resolve_sm_scale(sm_scale: float, head_dim: int) -> float:
    """Apply the reference's ``sm_scale == 0.0`` sentinel.

    ``kernel_flash2.cu:769-771`` / ``kernel_naive.cu:278-280``: an explicit
    0.0 means ``1.0f / sqrtf(float(D))``, computed in float32 and widened to
    double.
    """
    if sm_scale == 0.0:
        return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    return float(sm_scale)


def sm_scale_log2(sm_scale: float) -> np.float32:
    """``float(sm_scale * LOG2_E)`` as in ``kernel_flash2.cu:772``.

    The reference's ``LOG2_E`` is a ``float`` constant (``:16``) multiplied
    by a ``double`` scale, so the product uses float(log2 e) widened to
    double before the final rounding to float.
    """
    return np.float32(float(sm_scale) * float(np.float32(LOG2_E)))


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    """Row softmax; a row of only -inf (no visible key) gives zeros."""
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0).astype(s.dtype)
    p = np.exp(s - m)
    tot = np.sum(p, axis=-1, keepdims=True)
    return p / np.where(tot > 0, tot, 1.0).astype(s.dtype)


def causal_visible(rows, nq: int, nk: int) -> np.ndarray:
    """Boolean [len(rows), nk]: key j visible to query i iff j <= i + nk - nq
    (top-left when nk == nq)."""
    rows = np.asarray(rows, dtype=np.int64)
    return np.arange(nk)[None, :] <= rows[:, None] + (nk - nq)


def _attention(q, k, v, sm_scale, causal, dtype, row_chunk, rows):
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must be 4-D [B, H, N, D]")
    b, h, nq, d = q.shape
    nk = k.shape[2]
    if k.shape != (b, h, nk, d) or v.shape != (b, h, nk, d):
        raise ValueError("k and v must be [B, H, N_k, D] matching q")
    rows = np.arange(nq) if rows is None else np.asarray(rows, dtype=np.int64)
    scale = dtype(resolve_sm_scale(sm_scale, d))
    out = np.empty((b, h, len(rows), d), dtype=dtype)
    kt = np.swapaxes(k.astype(dtype), -1, -2)  # [B, H, D, N_k]
    vv = v.astype(dtype)
    for c0 in range(0, len(rows), row_chunk):
        sel = rows[c0:c0 + row_chunk]
        qq = q[:, :, sel, :].astype(dtype)
        s = np.matmul(qq, kt) * scale  # [B, H, rows, N_k]
        if causal:
            s = np.where(causal_visible(sel, nq, nk), s, dtype(-np.inf))
        p = _softmax_rows(s)
        out[:, :, c0:c0 + len(sel), :] = np.matmul(p, vv)
    return out


def _chunk(q, k, budget):
    b, h = q.shape[:2]
    nk = k.shape[2]
    return max(1, budget // max(1, b * h * nk))


def attention_fp32(q, k, v, sm_scale=0.0, causal=False, rows=None, row_chunk=None):
    """softmax(Q.K^T * sm_scale [+ causal mask]) . V evaluated in float32.

    Inputs are any float arrays [B, H, N, D] (normally fp16); they are
    upcast once.  ``rows`` restricts the evaluation to those query indices
    (the result is then [B, H, len(rows), D]); the causal mask still uses
    each row's true index.  Rows are processed in chunks so the score block
    stays below ~256 MiB even at N=16384.
    """
    if row_chunk is None:
        row_chunk = _chunk(q, k, 64 << 20)
    return _attention(q, k, v, sm_scale, causal, np.float32, row_chunk, rows)


def attention_fp64(q, k, v, sm_scale=0.0, causal=False, rows=None, row_chunk=None):
    """Same as :func:`attention_fp32` in float64 (cross-check only)."""
    if row_chunk is None:
        row_chunk = _chunk(q, k, 32 << 20)
    return _attention(q, k, v, sm_scale, causal, np.float64, row_chunk, rows)


def attention_lse(q, k, sm_scale=0.0, causal=False, dtype=np.float64):
    """Per-row log-sum-exp [B, H, N_q] of the scaled (and masked) scores,
    natural log; -inf for a row with no visible key."""
    b, h, nq, d = q.shape
    nk = k.shape[2]
    scale = dtype(resolve_sm_scale(sm_scale, d))
    s = np.matmul(q.astype(dtype), np.swapaxes(k.astype(dtype), -1, -2)) * scale
    if causal:
        s = np.where(causal_visible(np.arange(nq), nq, nk), s, dtype(-np.inf))
    m = np.max(s, axis=-1)
    mf = np.where(np.isfinite(m), m, 0.0)
    tot = np.sum(np.exp(s - mf[..., None]), axis=-1)
    with np.errstate(divide="ignore"):
        return np.where(tot > 0, mf + np.log(tot), -np.inf)


def attention_bruteforce(q, k, v, sm_scale=0.0, causal=False):
    """Scalar float64 loops, one query at a time (tiny shapes only).

    Written independently of the vectorised path: an explicit dot product
    per (query, key), ``math.exp`` after subtracting the visible-row max,
    then the weighted sum of V rows.
    """
    b, h, nq, d = q.shape
    nk = k.shape[2]
    scale = resolve_sm_scale(sm_scale, d)
    qf = q.astype(np.float64).tolist()
    kf = k.astype(np.float64).tolist()
    vf = v.astype(np.float64).tolist()
    out = np.zeros((b, h, nq, d), dtype=np.float64)
    for bi in range(b):
        for hi in range(h):
            for i in range(nq):
                visible = range(max(0, min(nk, i + 1 + nk - nq))) if causal else range(nk)
                if len(visible) == 0:
                    continue  # no visible key: the row stays 0
                logits = []
                for j in visible:
                    dot = 0.0
                    for t in range(d):
                        dot += qf[bi][hi][i][t] * kf[bi][hi][j][t]
                    logits.append(dot * scale)
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                tot = sum(w)
                for wj, j in zip(w, visible):
                    for t in range(d):
                        out[bi, hi, i, t] += wj / tot * vf[bi][hi][j][t]
    return out


def attention_flops(batch, heads, seq, head_dim, causal):
    """``benchmark_throughput.py:23-31``: 4.B.H.N^2.D, halved when causal."""
    mult = 2.0 if causal else 4.0
    return mult * batch * heads * (seq ** 2) * head_dim


def attention_bytes(batch, heads, seq, head_dim, elem_bytes=2):
    """Algorithmic HBM bytes: Q, K, V read once and O written once."""
    return 4 * batch * heads * seq * head_dim * elem_bytes


def error_stats(out, ref):
    """(max-abs, mean-abs) of ``out - ref`` in float64."""
    diff = np.abs(np.asarray(out, dtype=np.float64) - np.asarray(ref, dtype=np.float64))
    if diff.size == 0:
        return 0.0, 0.0
    return float(diff.max()), float(diff.mean())
