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
were checked when it ran eagerly). Every layer of one forward receives the same
position_ids tensor, so the host read is made once per forward: the result is kept
for that tensor object while its contents are unchanged (its version counter).

Several queries per row (a prompt): bf16 queries that the engine's rule
(qwen3.use_prompt_kernel: more than 64 rows reaching past position 160) gives to the
causal prompt-attention kernel take it (egpt_prefill_attn: query t at position
pos0 + t attends slots 0..pos0 + t, one pass over the prefix per block of queries);
the others, and other dtypes, run as a batch of single queries of the split-K
decode kernel over the same cache (batch stride 0), query t attending slots
0..position_ids[b, t].
"""

import weakref

import torch

from . import _lib
from .decode_attention import _run
from .qwen3 import use_prompt_kernel

NAME = 'egpt_decode'

# The last position_ids / mask that passed the host check: (position_ids ref, its version, mask ref or None, mask
# version, (B, T, cap), host positions [B, T]).
_checked = [None]


def _cached_positions(position_ids, attention_mask, key):
    c = _checked[0]
    if c is None or position_ids is None:
        return None
    pref, pver, mref, mver, ckey, p = c
    if pref() is not position_ids or position_ids._version != pver or ckey != key:
        return None
    if attention_mask is None:
        return p if mref is None else None
    if mref is None or mref() is not attention_mask or attention_mask._version != mver:
        return None
    return p


def _remember(position_ids, attention_mask, key, p):
    if position_ids is None:
        return
    mref = None if attention_mask is None else weakref.ref(attention_mask)
    mver = None if attention_mask is None else attention_mask._version
    _checked[0] = (weakref.ref(position_ids), position_ids._version, mref, mver, key, p)


def query_slots(query, key, attention_mask=None, position_ids=None):
    """[B, T] int64: the last cache slot each query attends (it attends slots 0..that slot).

    Raises ValueError when the positions or the mask do not describe a causal prefix of the cache: rows at
    different positions (a padded batch), positions that are not consecutive within a row, positions outside
    the cache, or a mask that hides a slot at or before a query's own or shows one after it."""
    pos, _ = _query_slots(query, key, attention_mask, position_ids)
    return pos


def _query_slots(query, key, attention_mask, position_ids):
    """(device positions [B, T], host positions [B, T] or None while a graph is being captured)."""
    b, _, t, _ = query.shape
    cap = key.shape[2]
    if position_ids is None:  # no positions: the queries are the last T slots of the cache
        pos = torch.arange(cap - t, cap, device=query.device).expand(b, t)
        p = torch.arange(cap - t, cap).expand(b, t)
    else:
        pos = position_ids.to(torch.long).expand(b, t)
        p = None
    if query.is_cuda and torch.cuda.is_current_stream_capturing():
        return pos, None
    shape_key = (b, t, cap)
    cached = _cached_positions(position_ids, attention_mask, shape_key)
    if cached is not None:
        return pos, cached
    if p is None:
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
    _remember(position_ids, attention_mask, shape_key, p)
    return pos, p


def _prompt_rows(query, key, value, row, pos0, scale):
    """Attention of row `row`'s T queries at positions pos0.. on the prompt kernel: [T, Hq, D], or None when the
    kernel does not take the operands (then the caller runs the decode kernel)."""
    _, hq, t, d = query.shape
    _, hkv, cap, _ = key.shape
    q = query[row].transpose(0, 1).contiguous()  # [T, Hq, D]
    k, v = key[row], value[row]
    if k.stride(2) != 1 or v.stride() != k.stride():
        return None
    out = torch.empty_like(q)
    st = _lib.lib().egpt_prefill_attn(q.data_ptr(), hq * d, k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                                      out.data_ptr(), hq * d, t, hq, hkv, d, cap, pos0, scale,
                                      _lib.stream_ptr(q.device))
    if st == _lib.EGPT_ERR_UNSUPPORTED:
        return None
    _lib.check('egpt_prefill_attn', st)
    return out


def egpt_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, position_ids=None,
                   **kwargs):
    """query [B, Hq, T, D], key/value [B, Hkv, L, D] -> ([B, T, Hq, D], None)."""
    b, hq, t, d = query.shape
    pos_all, host = _query_slots(query, key, attention_mask, position_ids)
    scale = scaling if scaling is not None else d ** -0.5
    outs = []
    for row in range(b):
        if host is not None and query.dtype == torch.bfloat16 and use_prompt_kernel(t, int(host[row, 0])):
            o = _prompt_rows(query, key, value, row, int(host[row, 0]), scale)
            if o is not None:
                outs.append(o)
                continue
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
