"""Readers of the golden fixtures in tests/golden/ (written by tests/golden/make_golden.py)."""

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def _cases(fname):
    z = np.load(os.path.join(GOLDEN, fname))
    for i in range(int(z['n_cases'])):
        p = f'c{i}_'
        yield {k[len(p):]: z[k] for k in z.files if k.startswith(p)}


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def linear_cases():
    """dicts: shape (M, N, K), x / w (bf16 bits), q int8, s fp32, truth fp64, rule (bf16 bits)."""
    return list(_cases('int8_linear.npz'))


def attention_cases():
    """dicts: shape (B, Hq, Hkv, cap, D), dtype, q [B, Hq, D] / k / v [B, Hkv, cap, D] (fp32 or bf16 bits),
    pos [B], truth fp64 [B, Hq, D]."""
    out = []
    for c in _cases('decode_attention.npz'):
        conv = (lambda a: a) if str(c['dtype']) == 'float32' else bf16_to_f32
        for n in ('q', 'k', 'v'):
            c[n] = conv(c[n]).astype(np.float32)
        out.append(c)
    return out


def tiny_greedy():
    with open(os.path.join(GOLDEN, 'qwen3_tiny_greedy.json')) as f:
        return json.load(f)


def bf16_ulp(a):
    """Spacing of bf16 numbers at |a| (elementwise; the smallest normal spacing near 0)."""
    a = np.maximum(np.abs(np.asarray(a, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(a)) - 7)

