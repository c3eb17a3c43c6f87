"""Writes the golden fixtures of this directory.

    python tests/golden/make_golden.py          (CPU; needs transformers for the Qwen3 tokens)

Every expected output here is computed from a formula that is independent of
oracle/ and of the HIP library, so the fixtures pin both:

* int8_linear.npz - per-output-channel int8 quantisation of bf16 weights in the reference's
  closed form (research/realmodel/int8_linear.py:106-117) and, per case, the fp64 truth
  x.double() @ (q.double() * s).T (research/realmodel/test_int8_linear.py:25) plus the output
  of the reference's rule for the row count (int8_linear.py:88-98: <= 16 rows, fp32 sum then
  scale then one bf16 rounding; more rows, bf16 GEMM of q's bf16 image, scale in fp32, bf16),
  in torch's own CPU matmul. Shapes follow the reference's tests (3 x 100 x 70 brute-force shape,
  test_int8_linear.py:32) plus aligned and 16/17-row boundary cases.
* decode_attention.npz - masked GQA decode attention as torch's fp64 scaled_dot_product_attention
  over slots 0..position, query head h reading kv head h // (Hq / Hkv)
  (research/kernelagent/tasks.py:34-40 with the kv heads repeated per group).
* qwen3_tiny_greedy.json - greedy tokens of transformers' Qwen3ForCausalLM on the
  reference's tiny test model (research/realmodel/test_fast_decode.py:9-15: seed 0,
  initializer_range 0.2, 4 query / 2 kv heads) with every linear and the lm_head quantised
  as the reference's quantize_model does (int8_linear.py:137-157), the int8 rule above in
  each linear, and attention in fp32 over the cache (the decode kernel's contract);
  prompts of 1, 5 and 37 tokens from Generator(seed 1), 40 new tokens each, as in
  test_fast_decode.py:26-40. The weights are not stored: tiny_model() rebuilds them
  from the seed, and the fixture keeps their sha256 so a drift is caught.
"""

import hashlib
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

LINEAR_CASES = [  # (rows, N, K, seed)
    (1, 64, 96, 0),
    (3, 100, 70, 1),
    (1, 128, 512, 2),
    (4, 48, 1000, 3),
    (16, 48, 64, 4),
    (17, 48, 64, 5),
]

ATTN_CASES = [  # (B, Hq, Hkv, cap, D, positions, dtype, seed)
    (2, 4, 2, 40, 64, [0, 31], 'float32', 0),
    (1, 16, 8, 40, 128, [38], 'bfloat16', 1),
    (2, 8, 8, 33, 64, [5, 32], 'bfloat16', 2),
]

TINY_PROMPTS = (1, 5, 37)
TINY_NEW_TOKENS = 40


def quantize_reference(w):
    """Per-output-channel symmetric int8 in the reference's closed form: s = max|w| / 127 (>= 1e-12), q = round(w / s)."""
    wf = w.float()
    s = (wf.abs().amax(1) / 127.0).clamp_min(1e-12)
    q = torch.round(wf / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


def int8_rule(x, q, s):
    """The reference's int8 linear for a bf16 row block x [M, K]."""
    if x.shape[0] <= 16:
        return (x.float() @ q.float().t() * s).to(torch.bfloat16)
    return ((x @ q.to(torch.bfloat16).t()).float() * s).to(torch.bfloat16)


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def linear_fixture():
    out = {}
    for i, (m, n, k, seed) in enumerate(LINEAR_CASES):
        g = torch.Generator().manual_seed(100 + seed)
        w = torch.randn(n, k, generator=g) * 0.05
        w[0, : min(k, 8)] *= 40.0  # one row with outliers: a large scale
        w = w.to(torch.bfloat16)  # quantised from bf16 model weights, as the reference does
        x = torch.randn(m, k, generator=g).to(torch.bfloat16)
        q, s = quantize_reference(w)
        truth = x.double() @ (q.double() * s.double()[:, None]).t()
        out[f'c{i}_shape'] = np.array([m, n, k])
        out[f'c{i}_x'] = bf16_bits(x)
        out[f'c{i}_w'] = bf16_bits(w)
        out[f'c{i}_q'] = q.numpy()
        out[f'c{i}_s'] = s.numpy()
        out[f'c{i}_truth'] = truth.numpy()
        out[f'c{i}_rule'] = bf16_bits(int8_rule(x, q, s))
    np.savez_compressed(os.path.join(HERE, 'int8_linear.npz'), n_cases=len(LINEAR_CASES), **out)


def attention_truth_f64(q, k, v, pos, scale):
    """q [B, Hq, D], k/v [B, Hkv, cap, D] (float64 tensors), pos [B]: torch's fp64 SDPA with kv heads
    repeated per group and a mask that keeps slots 0..pos[b] -> [B, Hq, D]."""
    hq, hkv, cap = q.shape[1], k.shape[1], k.shape[2]
    kk = k.repeat_interleave(hq // hkv, 1)
    vv = v.repeat_interleave(hq // hkv, 1)
    keep = torch.arange(cap)[None, :] <= torch.as_tensor(pos)[:, None]  # [B, cap]
    out = torch.nn.functional.scaled_dot_product_attention(q[:, :, None], kk, vv, attn_mask=keep[:, None, None, :],
                                                           scale=scale)
    return out[:, :, 0]


def attention_fixture():
    out = {}
    for i, (b, hq, hkv, cap, d, pos, dtype, seed) in enumerate(ATTN_CASES):
        g = torch.Generator().manual_seed(200 + seed)
        dt = getattr(torch, dtype)
        q = torch.randn(b, hq, d, generator=g).to(dt)
        k = torch.randn(b, hkv, cap, d, generator=g).to(dt)
        v = torch.randn(b, hkv, cap, d, generator=g).to(dt)
        p = np.array(pos, dtype=np.int64)
        truth = attention_truth_f64(q.double(), k.double(), v.double(), p, d ** -0.5).numpy()
        out[f'c{i}_shape'] = np.array([b, hq, hkv, cap, d])
        out[f'c{i}_dtype'] = np.array(dtype)
        for name, t in (('q', q), ('k', k), ('v', v)):
            out[f'c{i}_{name}'] = t.numpy() if dtype == 'float32' else bf16_bits(t)
        out[f'c{i}_pos'] = p
        out[f'c{i}_truth'] = truth
    np.savez_compressed(os.path.join(HERE, 'decode_attention.npz'), n_cases=len(ATTN_CASES), **out)


# ------------------------------------------------------------------ tiny Qwen3

def tiny_model():
    """The reference's tiny Qwen3 (test_fast_decode.py:9-15), bf16, on the CPU."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=32, max_position_embeddings=256, tie_word_embeddings=True,
                      initializer_range=0.2)
    return Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


def quantized_state(model):
    """State dict with every decoder linear and the lm_head as `<name>.qweight` / `<name>.scale`
    (the tied lm_head becomes an int8 copy of the embedding; embedding and norms stay bf16)."""
    sd = {k: v.detach().clone() for k, v in model.state_dict().items()}
    out = {}
    for name, t in sd.items():
        base = name[:-len('.weight')] if name.endswith('.weight') else None
        if base and (base.endswith(('_proj',)) or base == 'lm_head'):
            out[base + '.qweight'], out[base + '.scale'] = quantize_reference(t)
        else:
            out[name] = t
    if 'lm_head.qweight' not in out:
        out['lm_head.qweight'], out['lm_head.scale'] = quantize_reference(sd['model.embed_tokens.weight'])
    return out


def state_sha256(state):
    h = hashlib.sha256()
    for name in sorted(state):
        t = state[name].contiguous()
        h.update(name.encode())
        h.update(str(t.dtype).encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.int8 else t.numpy().tobytes())
    return h.hexdigest()


def tiny_prompts():
    g = torch.Generator().manual_seed(1)
    return [torch.randint(0, 512, (p,), generator=g).tolist() for p in TINY_PROMPTS]


class _Int8Rule(torch.nn.Module):
    def __init__(self, q, s):
        super().__init__()
        self.q, self.s = q, s

    def forward(self, x):
        k = x.shape[-1]
        return int8_rule(x.reshape(-1, k), self.q, self.s).reshape(*x.shape[:-1], self.q.shape[0])


def _fp32_cache_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """fp32 attention over the cache, causal for multi-row blocks; the result in the activation dtype."""
    g = query.shape[1] // key.shape[1]
    k = key.float().repeat_interleave(g, 1)
    v = value.float().repeat_interleave(g, 1)
    s = (query.float() @ k.transpose(-1, -2)) * scaling
    t, n = s.shape[-2], s.shape[-1]
    allowed = torch.arange(n)[None, :] <= (n - t + torch.arange(t))[:, None]
    s = s.masked_fill(~allowed, float('-inf'))
    return (torch.softmax(s, -1) @ v).to(query.dtype).transpose(1, 2).contiguous(), None


@torch.no_grad()
def tiny_fixture():
    import transformers
    transformers.AttentionInterface.register('golden_fp32_cache', _fp32_cache_attention)
    model = tiny_model()
    state = quantized_state(model)
    model.config._attn_implementation = 'golden_fp32_cache'
    for name, mod in list(model.named_modules()):
        if isinstance(mod, torch.nn.Linear):
            parent_name, _, child = name.rpartition('.')
            parent = model.get_submodule(parent_name) if parent_name else model
            setattr(parent, child, _Int8Rule(state[name + '.qweight'], state[name + '.scale']))
    runs = []
    for prompt in tiny_prompts():
        x = torch.tensor([prompt])
        res = model.generate(input_ids=x, attention_mask=torch.ones_like(x), max_new_tokens=TINY_NEW_TOKENS,
                             min_new_tokens=TINY_NEW_TOKENS, do_sample=False, pad_token_id=0, output_logits=True,
                             return_dict_in_generate=True)
        toks = res.sequences[0, len(prompt):].tolist()
        margins, tops = [], []
        for lg in res.logits:
            top2 = torch.topk(lg[0].float(), 2).values
            tops.append(float(top2[0]))
            margins.append(float(top2[0] - top2[1]))
        runs.append({'prompt': prompt, 'tokens': toks, 'margins': margins, 'tops': tops})
    cfg = model.config
    rope = getattr(cfg, 'rope_parameters', None) or {}
    fixture = {
        'model': 'transformers Qwen3ForCausalLM, test_fast_decode.py:9-15 tiny config, torch.manual_seed(0), bf16',
        'transformers': transformers.__version__,
        'torch': torch.__version__.split('+')[0],
        'rope_theta': float(rope.get('rope_theta', getattr(cfg, 'rope_theta', 0.0))),
        'rms_eps': float(cfg.rms_norm_eps),
        'weights_sha256': state_sha256(state),
        'new_tokens': TINY_NEW_TOKENS,
        'runs': runs,
    }
    with open(os.path.join(HERE, 'qwen3_tiny_greedy.json'), 'w') as f:
        json.dump(fixture, f, indent=1)


if __name__ == '__main__':
    linear_fixture()
    attention_fixture()
    tiny_fixture()
    for f in sorted(os.listdir(HERE)):
        if not f.endswith('.py'):
            print(f, os.path.getsize(os.path.join(HERE, f)), 'bytes')
