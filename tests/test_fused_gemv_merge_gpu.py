"""The split-K merge in the fused GEMV's prologue (egpt_int8_gemv_fused with attention partials), at split
counts on both sides of every unroll bound the launch picks (4, 8, 16), with empty trailing splits.

The merge is the combine of the reference's split-K decode attention (research/phase5/decode_attention.py:59-71):
w_s = exp(m_s - max m), h = bf16(sum_s w_s acc_s / sum_s w_s l_s), empty splits (m = -inf) weighing 0. The weights
here are a scaled identity (row n reads column n only), so the GEMV returns the merged row itself and each element
is checked against an fp64 evaluation of that formula.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HEADS, D = 16, 128
K = HEADS * D


def bf16_ulp(v):
    a = np.abs(np.asarray(v, np.float64))
    a = np.where(a == 0, 1e-38, a)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def partials(nsplit, empty, seed):
    """Partial states of HEADS heads over nsplit splits, the last `empty` of them empty. The last live split
    holds the largest m, so counting it twice (or dropping it) moves every merged element."""
    g = np.random.default_rng(seed)
    m = g.normal(0.0, 2.0, (HEADS, nsplit)).astype(np.float32)
    live = nsplit - empty
    m[:, live - 1] = m[:, :live].max(axis=1) + 0.5
    l = g.uniform(0.5, 8.0, (HEADS, nsplit)).astype(np.float32)
    acc = (l[:, :, None] * g.normal(0.0, 1.0, (HEADS, nsplit, D))).astype(np.float32)
    m[:, live:] = -np.inf
    l[:, live:] = 0.0
    acc[:, live:] = 0.0
    return m, l, acc


def merged_fp64(m, l, acc):
    m64, l64, a64 = m.astype(np.float64), l.astype(np.float64), acc.astype(np.float64)
    mx = m64.max(axis=1, keepdims=True)
    w = np.where(np.isneginf(m64), 0.0, np.exp(m64 - mx))
    return ((w[:, :, None] * a64).sum(axis=1) / (w * l64).sum(axis=1, keepdims=True)).reshape(-1)


@pytest.mark.parametrize('nsplit,empty', [(1, 0), (2, 1), (3, 0), (4, 0), (4, 2), (5, 0), (7, 0), (8, 3),
                                          (9, 0), (11, 4), (13, 0), (16, 0), (16, 5)])
def test_merge_prologue_matches_combine(nsplit, empty):
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    m, l, acc = partials(nsplit, empty, seed=100 + nsplit * 7 + empty)
    want = merged_fp64(m, l, acc)
    dev = 'cuda'
    # the workspace layout of egpt_decode_attn for one row: m[h, s], l[h, s], acc[h, s, d]
    tm = torch.from_numpy(m).to(dev)
    tl = torch.from_numpy(l).to(dev)
    ta = torch.from_numpy(acc).to(dev)
    q = torch.zeros(K, K, dtype=torch.int8)
    q.fill_diagonal_(64)
    q = q.to(dev)
    s = torch.full((K,), 1.0 / 64.0, dtype=torch.float32, device=dev)
    resid = torch.zeros(K, dtype=torch.bfloat16, device=dev)
    y = torch.empty(K, dtype=torch.bfloat16, device=dev)
    d = _lib.GemvFused()
    d.epilogue, d.N, d.K = _lib.EPI_RESIDUAL, K, K
    d.merge_m, d.merge_l, d.merge_acc = tm.data_ptr(), tl.data_ptr(), ta.data_ptr()
    d.merge_splits, d.head_dim = nsplit, D
    d.w, d.ldw, d.scale = q.data_ptr(), K, s.data_ptr()
    d.y, d.resid = y.data_ptr(), resid.data_ptr()
    _lib.check('egpt_int8_gemv_fused', lib.egpt_int8_gemv_fused(ctypes.byref(d), None))
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    # one bf16 rounding of the merged value, a second of the GEMV output, and the GEMV's fp32 sum over the
    # row (a biased sum of 2048 terms of size 128 |h|: about 2^-24 sqrt(K) 128 max|h| absolute)
    sum_err = 2.0 ** -24 * np.sqrt(K) * 128.0 * np.abs(want).max() / 64.0 * 16.0
    bound = 2.0 * bf16_ulp(want) + sum_err
    diff = np.abs(got - want)
    assert np.all(diff <= bound), (float((diff - bound).max()), int(np.argmax(diff - bound)))
    near = np.abs(got - want) <= bf16_ulp(want) / 2 + sum_err
    assert near.mean() >= 0.99, float(near.mean())


def test_merge_prologue_refuses_more_than_16_splits():
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    d = _lib.GemvFused()
    dev = 'cuda'
    buf = torch.zeros(HEADS * 17 * (D + 2), dtype=torch.float32, device=dev)
    q = torch.zeros(K, K, dtype=torch.int8, device=dev)
    s = torch.ones(K, dtype=torch.float32, device=dev)
    y = torch.empty(K, dtype=torch.bfloat16, device=dev)
    d.epilogue, d.N, d.K = _lib.EPI_RESIDUAL, K, K
    d.merge_m, d.merge_l, d.merge_acc = buf.data_ptr(), buf.data_ptr(), buf.data_ptr()
    d.merge_splits, d.head_dim = 17, D
    d.w, d.ldw, d.scale, d.y, d.resid = q.data_ptr(), K, s.data_ptr(), y.data_ptr(), y.data_ptr()
    assert lib.egpt_int8_gemv_fused(ctypes.byref(d), None) != 0
