"""On-disk int8 weights for the Qwen3 decode engine (safetensors), loaded without re-quantising.

The reference quantises the bf16 checkpoint on every load (research/realmodel/int8_linear.py:137-157:
quantize_model walks every nn.Linear and calls quantize_weight). This format stores the result once,
already in the engine's device layout, so loading is a read plus a host-to-device copy:

  layers.{i}.qkv.qweight      int8 [(Hq + 2 Hkv) * D, hidden]   q, k, v rows stacked
  layers.{i}.qkv.scale        fp32 [(Hq + 2 Hkv) * D]
  layers.{i}.o.qweight/scale          [hidden, Hq * D]
  layers.{i}.gate_up.qweight/scale    [2 * inter, hidden]       gate rows then up rows
  layers.{i}.down.qweight/scale       [hidden, inter]
  layers.{i}.input_norm, .post_norm, .q_norm, .k_norm   bf16
  embed        bf16 [vocab, hidden]
  final_norm   bf16 [hidden]
  lm_head.qweight/scale   int8 [vocab, hidden] / fp32 (a tied head: the int8 copy of the embedding)
  rope.inv_freq           fp32 [head_dim / 2]   (present when the model carried its own)

The safetensors header metadata holds `format` (FORMAT) and `config` (the Qwen3Config fields as JSON).
Rows are [N, K] row-major, the nn.Linear layout the kernels stream; scales are per output row.
"""

import dataclasses
import json

import torch

FORMAT = 'efficientgpt-mi355x-qwen3-int8/1'

_LINEARS = (('qkv', 'qkv_q', 'qkv_s'), ('o', 'o_q', 'o_s'), ('gate_up', 'gu_q', 'gu_s'), ('down', 'down_q', 'down_s'))
_NORMS = (('input_norm', 'in_w'), ('post_norm', 'post_w'), ('q_norm', 'qn_w'), ('k_norm', 'kn_w'))


def _tensors(packed, inv_freq=None):
    out = {}
    for i, L in enumerate(packed['layers']):
        for name, q, s in _LINEARS:
            out[f'layers.{i}.{name}.qweight'] = L[q]
            out[f'layers.{i}.{name}.scale'] = L[s]
        for name, key in _NORMS:
            out[f'layers.{i}.{name}'] = L[key]
    out['embed'] = packed['embed']
    out['final_norm'] = packed['norm_w']
    out['lm_head.qweight'] = packed['head_q']
    out['lm_head.scale'] = packed['head_s']
    if inv_freq is not None:
        out['rope.inv_freq'] = inv_freq.detach().float()
    return {k: v.detach().contiguous().cpu() for k, v in out.items()}


def save_int8(path, cfg, packed, inv_freq=None):
    """Write a packed layout (efficientgpt_amd.qwen3.pack_qwen3) and its config to `path`."""
    from safetensors.torch import save_file
    meta = {'format': FORMAT, 'config': json.dumps(dataclasses.asdict(cfg))}
    save_file(_tensors(packed, inv_freq), path, metadata=meta)


def save_engine(path, engine):
    """Write the weights a Qwen3Int8Engine holds (device tensors are copied to the host)."""
    packed = {'layers': engine.layers, 'embed': engine.embed, 'norm_w': engine.norm_w,
              'head_q': engine.head_q, 'head_s': engine.head_s}
    save_int8(path, engine.cfg, packed, engine.inv_freq)


def load_int8(path, device='cpu'):
    """(Qwen3Config, packed layout, inv_freq or None) from `path`; raises ValueError on a foreign file."""
    from safetensors import safe_open
    from .qwen3 import Qwen3Config, check_packed
    with safe_open(path, framework='pt', device=str(device)) as f:
        meta = f.metadata() or {}
        if meta.get('format') != FORMAT:
            raise ValueError(f'{path}: not an {FORMAT} checkpoint (format {meta.get("format")!r})')
        cfg = Qwen3Config(**json.loads(meta['config']))
        names = set(f.keys())
        get = f.get_tensor
        layers = []
        for i in range(cfg.layers):
            L = {}
            for name, q, s in _LINEARS:
                L[q] = get(f'layers.{i}.{name}.qweight')
                L[s] = get(f'layers.{i}.{name}.scale')
            for name, key in _NORMS:
                L[key] = get(f'layers.{i}.{name}')
            layers.append(L)
        packed = {'layers': layers, 'embed': get('embed'), 'norm_w': get('final_norm'),
                  'head_q': get('lm_head.qweight'), 'head_s': get('lm_head.scale')}
        inv_freq = get('rope.inv_freq') if 'rope.inv_freq' in names else None
    check_packed(cfg, packed)  # a truncated or mismatched file fails here
    return cfg, packed, inv_freq
