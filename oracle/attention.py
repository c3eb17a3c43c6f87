"""Masked GQA decode attention on the CPU (test infrastructure; see oracle/__init__.py).

  attention_truth      fp64 masked attention over slots 0..position[b]
                       (research/kernelagent/tasks.py:34-40, research/phase5/test_graph_gpu.py:221-224),
                       with K/V of kv head h // G serving query head h (repeat_kv semantics).
  attention_splitk     fp32 restatement of the reference's flash-decoding pair:
                       _split_kernel (research/phase5/decode_attention.py:31-56) per split of
                       SPLIT slots in BLOCK_N tiles, then _combine_kernel (:59-71).
  prefill_truth        fp64 causal attention of a prompt block (query row t at position pos0 + t)
                       over a static cache, the prompt pass of transformers' Qwen3 attention.
  bytes_moved          algorithmic bytes of one call (K and V rows read once, q read, out written).
Inputs are numpy arrays: q [B, Hq, 1, D], k/v [B, Hkv, cap, D], position int64 [1] or [B].
"""

import numpy as np


def _live(position, b, cap):
    pos = np.asarray(position).reshape(-1)
    p = int(pos[0] if pos.size == 1 else pos[b])
    return min(max(p, 0), cap - 1) + 1


def attention_truth(q, k, v, position, scale=None):
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    bsz, hq, one, d = q.shape
    hkv, cap = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    out = np.zeros((bsz, hq, 1, d))
    for b in range(bsz):
        n = _live(position, b, cap)
        for h in range(hq):
            kk = k[b, h // g, :n]
            s = (kk @ q[b, h, 0]) * scale
            p = np.exp(s - s.max())
            out[b, h, 0] = (p / p.sum()) @ v[b, h // g, :n]
    return out


def attention_splitk(q, k, v, position, split=16, block_n=16):
    """fp32 split-K online softmax with the reference's fixed split layout, then the combine."""
    f32 = np.float32
    q = np.asarray(q, f32)
    k = np.asarray(k, f32)
    v = np.asarray(v, f32)
    bsz, hq, one, d = q.shape
    hkv, cap = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = f32(d ** -0.5)
    nsplit = 1 << max(0, int(np.ceil(np.log2(-(-cap // split)))))  # next power of two, as the reference
    out = np.zeros((bsz, hq, 1, d), f32)
    for b in range(bsz):
        length = _live(position, b, cap)
        for h in range(hq):
            kk, vv, qq = k[b, h // g], v[b, h // g], q[b, h, 0]
            ms = np.full(nsplit, -np.inf, f32)
            ls = np.zeros(nsplit, f32)
            accs = np.zeros((nsplit, d), f32)
            for s_idx in range(nsplit):
                start, end = s_idx * split, min(s_idx * split + split, length)
                m_i, l_i, acc = f32(-np.inf), f32(0), np.zeros(d, f32)
                for n0 in range(start, end, block_n):
                    n1 = min(n0 + block_n, end)
                    scores = (kk[n0:n1] @ qq).astype(f32) * scale
                    m_new = max(m_i, f32(scores.max()))
                    alpha = f32(np.exp(m_i - m_new))
                    p = np.exp(scores - m_new).astype(f32)
                    l_i = f32(l_i * alpha + p.sum(dtype=f32))
                    acc = (acc * alpha + (p[:, None] * vv[n0:n1]).sum(0, dtype=f32)).astype(f32)
                    m_i = m_new
                ms[s_idx], ls[s_idx], accs[s_idx] = m_i, l_i, acc
            w = np.exp(ms - ms.max()).astype(f32)  # empty splits: m = -inf -> weight 0
            out[b, h, 0] = (accs * w[:, None]).sum(0, dtype=f32) / (ls * w).sum(dtype=f32)
    return out


def prefill_truth(q, k, v, pos0, scale=None):
    """fp64 causal attention of a prompt block over a static cache (the prompt pass of transformers'
    Qwen3Attention.forward: SDPA with the causal mask over the cache, HF models/qwen3/modeling_qwen3.py:252-280,
    integrations/sdpa_attention.py:79-102). q [rows, Hq, D] holds query rows at positions pos0 + t; k, v
    [Hkv, cap, D]; row t of query head h attends slots 0 .. pos0 + t of kv head h // G. Returns [rows, Hq, D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    rows, hq, d = q.shape
    hkv = k.shape[0]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    n = pos0 + rows
    allowed = np.arange(n)[None, :] <= (pos0 + np.arange(rows))[:, None]  # [rows, n]
    out = np.zeros((rows, hq, d))
    for h in range(hq):
        s = (q[:, h] @ k[h // g, :n].T) * scale
        s = np.where(allowed, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ v[h // g, :n]
    return out


def bytes_moved(b, hq, hkv, live, d, elem_bytes=2):
    """K and V rows of every live slot read once per kv head, q read, out written."""
    return elem_bytes * (2 * b * hkv * live * d + 2 * b * hq * d)
