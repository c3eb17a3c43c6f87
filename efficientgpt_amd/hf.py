"""transformers attention-registry adapter: Qwen3 (and any GQA decoder) attention on the HIP kernel.

The reference's Qwen3 path reaches attention through transformers'
ALL_ATTENTION_FUNCTIONS (modeling_qwen3.py:262-276, integrations/sdpa_attention.py)
and scans the whole static cache with a mask. `register()` adds an implementation
named 'egpt_decode' that calls the split-K GQA kernel instead, reading only slots
0..position for each query (the position comes from `position_ids`, which
transformers forwards to the attention function). Select it with
`model.config._attn_implementation = 'egpt_decode'` or
`from_pretrained(..., attn_implementation='egpt_decode')`.

Prefill (several queries per row) is run as a batch of single queries over the
same cache (batch stride 0), query t attending to slots 0..position_ids[b, t].
"""

import torch

from .decode_attention import _run

NAME = 'egpt_decode'


def egpt_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, position_ids=None,
                   **kwargs):
    """query [B, Hq, T, D], key/value [B, Hkv, L, D] -> ([B, T, Hq, D], None)."""
    b, hq, t, d = query.shape
    if position_ids is None:  # no positions: the queries are the last T slots of the cache
        position_ids = torch.arange(key.shape[2] - t, key.shape[2], device=query.device).expand(b, t)
    scale = scaling if scaling is not None else d ** -0.5
    outs = []
    for row in range(b):
        q = query[row].transpose(0, 1).unsqueeze(2)  # [T, Hq, 1, D]
        k = key[row:row + 1].expand(t, -1, -1, -1)  # stride-0 batch over one cache row
        v = value[row:row + 1].expand(t, -1, -1, -1)
        pos = position_ids[row].reshape(-1).to(torch.long).contiguous()
        outs.append(_run(q, k, v, pos, 0, scale=scale).squeeze(2))  # [T, Hq, D]
    return torch.stack(outs, 0), None


def register():
    """Register 'egpt_decode' in transformers' attention registry (idempotent)."""
    from transformers import AttentionInterface
    AttentionInterface.register(NAME, egpt_attention)
    return NAME
