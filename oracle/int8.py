"""Weight-only int8 linear on the CPU (test infrastructure; see oracle/__init__.py).

Restates research/realmodel/int8_linear.py in numpy:
  quantize_weight       :106-117  (per-row symmetric, round half to even, clamp +-127)
  linear_decode         :26-38    (_dot16: fp32 sum, scale after the sum, one bf16 rounding)
  linear_prefill        :96-97    (bf16 GEMM output, times scale in fp32, bf16 again)
  linear_truth          research/realmodel/test_int8_linear.py:25 (fp64, exact dequantisation)
  linear_naive          research/realmodel/test_int8_linear.py:26 (bf16 dequant + bf16 GEMM)
  tolerance_vs_naive    research/realmodel/test_int8_linear.py:28-29
  tolerance_vs_eager    research/kernelagent/evaluate.py:91-99 with tasks.py:150-158, 206-212
Activations are float32 arrays holding bf16 values.
"""

import numpy as np

from .numerics import to_bf16

MAX_DECODE_ROWS = 16


def quantize_weight(w):
    """w float [N, K] -> (q int8 [N, K], s float32 [N]); s = max(max|w_row| / 127, 1e-12) in fp32."""
    wf = np.asarray(w, dtype=np.float32)
    amax = np.abs(wf).max(axis=1) if wf.shape[1] else np.zeros(wf.shape[0], np.float32)
    s = np.maximum(amax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    q = np.clip(np.rint(wf / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def _exact_dot_f32(x, q):
    """sum_k x[m, k] q[n, k] accumulated in fp64 (far finer than the kernels' fp32), rounded once to fp32."""
    return (np.asarray(x, np.float64) @ np.asarray(q, np.float64).T).astype(np.float32)


def linear_decode(x, q, s):
    """bf16( s[n] * fp32(sum_k x q) ): the decode kernel's contract, with the sum taken in fp64."""
    acc = _exact_dot_f32(x, q)
    return to_bf16(acc * np.asarray(s, np.float32)[None, :])


def linear_prefill(x, q, s):
    """bf16( fp32(bf16(x @ q^T)) * s ): the reference's row count > 16 path."""
    t = to_bf16(_exact_dot_f32(x, q))
    return to_bf16(t * np.asarray(s, np.float32)[None, :])


def linear(x, q, s):
    """The reference op's row rule: <= 16 rows take the decode kernel, more take the prefill formula."""
    rows = np.asarray(x).reshape(-1, np.asarray(x).shape[-1]).shape[0]
    return linear_decode(x, q, s) if rows <= MAX_DECODE_ROWS else linear_prefill(x, q, s)


def linear_truth(x, q, s):
    """fp64 x @ (q * s)^T with exact dequantisation."""
    w = np.asarray(q, np.float64) * np.asarray(s, np.float64)[:, None]
    return np.asarray(x, np.float64) @ w.T


def linear_naive(x, q, s):
    """x @ (q.bf16 * s.bf16)^T in bf16: what a dequantise-then-GEMM implementation returns."""
    w = to_bf16(np.asarray(q, np.float32) * to_bf16(np.asarray(s, np.float32))[:, None])
    return to_bf16(_exact_dot_f32(x, w))


def tolerance_vs_naive(x, q, s):
    """max(2 * err(naive), 1e-3), errors as max |.| against the fp64 truth."""
    truth = linear_truth(x, q, s)
    return max(2.0 * float(np.abs(linear_naive(x, q, s) - truth).max(initial=0.0)), 1e-3)


def tolerance_vs_eager(x, q, s, factor=4.0, floor=1e-3):
    """factor * err(eager bf16 dequant GEMM) + floor, the search harness's accept rule."""
    truth = linear_truth(x, q, s)
    return factor * float(np.abs(linear_naive(x, q, s) - truth).max(initial=0.0)) + floor


def max_err(y, x, q, s):
    return float(np.abs(np.asarray(y, np.float64) - linear_truth(x, q, s)).max(initial=0.0))


def bytes_moved(m, n, k):
    """Algorithmic bytes of one call: weights + scales + x + y (research/kernelagent/tasks.py:208-209)."""
    return n * k + 4 * n + 2 * m * k + 2 * m * n
