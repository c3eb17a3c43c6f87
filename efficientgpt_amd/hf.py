"""transformers attention-registry adapter: Qwen3 (and any GQA decoder) attention on the HIP kernel.

The reference's Qwen3 path reaches attention through transformers'
ALL_ATTENTION_FUNCTIONS (modeling_qwen3.py:262-276, integrations/sdpa_attention.py)
and scans the whole static cache with a mask. `register()` adds an implementation
named 'egpt_decode' that calls the split-K GQA kernel instead, reading only slots
0..position for each query. Select it with
`model.config._attn_implementation = 'egpt_decode'` or
`from_pretrained(..., attn_implementation='egpt_decode')`.

Which slots a query may read. The kernel reads a prefix of the cache, slots
0..position. transformers hands a registered attention function no mask of its own
making (attention_mask is None) but forwards `position_ids`, which for an unpadded
batch are the cache slots of the queries. A left-padded batch breaks that: its
position ids come from the padding mask (pads and the first real token share
position 0), the rows sit at different slots, and the pad slots would need masking
in the middle of the prefix. The adapter checks, before the kernel runs, that every
row holds the same consecutive positions inside the cache and that any mask it is
given allows exactly slots 0..position; anything else raises ValueError instead of
attending the wrong slots. The check reads the positions on the host, so it is
skipped while a graph is being captured (a captured step replays fixed shapes that
were checked when it ran eagerly).

Prefill (several queries per row) is run as a batch of single queries over the
same cache (batch stride 0), query t attending to slots 0..position_ids[b, t].
"""

import torch

from .decode_attention import _run

NAME = 'egpt_decode'


def query_slots(query, key, attention_mask=None, position_ids=None):
    """[B, T] int64: the last cache slot each query attends (it attends slots 0..that slot).

    Raises ValueError when the positions or the mask do not describe a causal prefix of the cache: rows at
    different positions (a padded batch), positions that are not consecutive within a row, positions outside
    the cache, or a mask that hides a slot at or before a query's own or shows one after it."""
    b, _, t, _ = query.shape
    cap = key.shape[2]
    if position_ids is None:  # no positions: the queries are the last T slots of the cache
        pos = torch.arange(cap - t, cap, device=query.device).expand(b, t)
    else:
        pos = position_ids.to(torch.long).expand(b, t)
    if query.is_cuda and torch.cuda.is_current_stream_capturing():
        return pos
    p = pos.cpu()
    if bool((p != p[:1]).any()):
        raise ValueError('egpt_decode attention: the rows of the batch sit at different positions (a padded '
                         'batch); it reads cache slots 0..position and cannot mask padding: use sdpa for padded '
                         'batches')
    if t > 1 and bool((p[:, 1:] - p[:, :-1] != 1).any()):
        raise ValueError('egpt_decode attention: position_ids are not consecutive within a row (left padding); '
                         'use sdpa for padded batches')
    if int(p.min()) < 0 or int(p.max()) >= cap:
        raise ValueError(f'egpt_decode attention: positions {int(p.min())}..{int(p.max())} outside the cache of '
                         f'{cap} slots')
    if attention_mask is not None:
        allowed = attention_mask if attention_mask.dtype == torch.bool else attention_mask == 0
        allowed = allowed.cpu()
        slots = torch.arange(allowed.shape[-1])
        want = slots[None, None, None, :] <= p[:, None, :, None]
        if not bool((allowed == want).all()):
            raise ValueError('egpt_decode attention: the attention mask is not the causal prefix 0..position of '
                             'every query (padding or a custom mask); use sdpa for such masks')
    return pos


def egpt_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, position_ids=None,
                   **kwargs):
    """query [B, Hq, T, D], key/value [B, Hkv, L, D] -> ([B, T, Hq, D], None)."""
    b, hq, t, d = query.shape
    pos_all = query_slots(query, key, attention_mask, position_ids)
    scale = scaling if scaling is not None else d ** -0.5
    outs = []
    for row in range(b):
        q = query[row].transpose(0, 1).unsqueeze(2)  # [T, Hq, 1, D]
        k = key[row:row + 1].expand(t, -1, -1, -1)  # stride-0 batch over one cache row
        v = value[row:row + 1].expand(t, -1, -1, -1)
        pos = pos_all[row].reshape(-1).contiguous()
        outs.append(_run(q, k, v, pos, 0, scale=scale).squeeze(2))  # [T, Hq, D]
    return torch.stack(outs, 0), None


def register():
    """Register 'egpt_decode' in transformers' attention registry (idempotent)."""
    from transformers import AttentionInterface
    AttentionInterface.register(NAME, egpt_attention)
    return NAME
