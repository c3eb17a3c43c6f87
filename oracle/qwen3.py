"""Qwen3 decoder with int8 linears, in torch on the CPU (test infrastructure; see oracle/__init__.py).

Follows transformers' Qwen3 (models/qwen3/modeling_qwen3.py: Qwen3RMSNorm :30-46,
rotary :80-136 and apply_rotary_pos_emb :139-166, Qwen3Attention :211-280,
Qwen3MLP :49-62, decoder layer :285-322, final norm + lm_head with
logits_to_keep=1) in the activation dtype of the model (bf16 or fp32), with every
linear replaced by the reference's int8 rule (research/realmodel/int8_linear.py:88-98:
<= 16 rows -> fp32 sum, scale, one bf16 rounding; more rows -> bf16 GEMM, scale,
bf16 again) and a tied lm_head quantised from the embedding
(research/realmodel/int8_linear.py:137-157). Attention is fp32 math over slots
0..position (the decode kernel's contract) with the result in the activation dtype.

Weights are a dict keyed by transformers' state-dict names; int8 linears hold
`<name>.qweight` (int8 [N, K]) and `<name>.scale` (fp32 [N]) instead of `<name>.weight`.
"""

from dataclasses import dataclass

import torch
import torch.nn.functional as F

MAX_DECODE_ROWS = 16
LINEARS = ('self_attn.q_proj', 'self_attn.k_proj', 'self_attn.v_proj', 'self_attn.o_proj',
           'mlp.gate_proj', 'mlp.up_proj', 'mlp.down_proj')


@dataclass(frozen=True)
class Qwen3Shape:
    vocab: int
    hidden: int
    inter: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    tied: bool = True


QWEN3_1_7B = Qwen3Shape(vocab=151936, hidden=2048, inter=6144, layers=28, heads=16, kv_heads=8, head_dim=128)
QWEN3_8B = Qwen3Shape(vocab=151936, hidden=4096, inter=12288, layers=36, heads=32, kv_heads=8, head_dim=128,
                      tied=False)
# research/realmodel/test_fast_decode.py:9-15 (transformers' default rope theta for this config: 1e4)
TINY = Qwen3Shape(vocab=512, hidden=128, inter=256, layers=2, heads=4, kv_heads=2, head_dim=32, rope_theta=1e4)


def quantize_rows(w):
    """Per-row symmetric int8 of a float matrix (research/realmodel/int8_linear.py:106-117), in torch."""
    wf = w.float()
    s = (wf.abs().amax(1) / 127.0).clamp_min(1e-12)
    q = torch.round(wf / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


def default_inv_freq(shape):
    """RoPE inverse frequencies in fp32 (modeling_qwen3.py:113-122)."""
    d = shape.head_dim
    return 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))


def rope_tables(shape, length, dtype, inv_freq=None):
    """cos / sin [length, head_dim] as transformers builds them: fp32 products and cos/sin, cast to `dtype`.

    `inv_freq` defaults to the fp32 formula; a model cast with `.to(torch.bfloat16)`
    carries a bf16-rounded copy, which callers pass in to match it.
    """
    inv_freq = default_inv_freq(shape) if inv_freq is None else inv_freq.detach().cpu().float()
    pos = torch.arange(length, dtype=torch.float)
    freqs = (inv_freq[None, :, None] @ pos[None, None, :]).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rms_norm(x, weight, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(x.dtype)


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


class Linear:
    """A float weight, or int8 codes + fp32 scales applied by the reference's row rule.

    `ksplit` > 1 takes the decode formula's fp32 sum the way the reference's split-K
    GEMV does (research/realmodel/int8_linear.py:41-64, :79-80): partial sums over
    chunks of KCHUNK = ceil(ceil(K / ksplit) / 128) * 128 columns, added in chunk
    order, then scaled and rounded once. It is the same product summed in another
    valid fp32 order, which is what tests use it for: two forms of the reference's own
    arithmetic whose difference measures how far rounding alone moves a result.
    """

    def __init__(self, weight=None, qweight=None, scale=None, ksplit=1):
        self.weight = weight
        self.q = qweight
        self.s = scale
        self.ksplit = ksplit
        self._qf = None

    def _sum(self, x):
        """fp32 x @ q^T, in one product or by the split-K chunks."""
        xf = x.float()
        k = xf.shape[-1]
        if self.ksplit <= 1:
            return xf @ self._qf.t()
        kchunk = -(-(-(-k // self.ksplit)) // 128) * 128
        acc = None
        for k0 in range(0, k, kchunk):
            part = xf[..., k0:k0 + kchunk] @ self._qf[:, k0:k0 + kchunk].t()
            acc = part if acc is None else acc + part
        return acc

    def __call__(self, x, rule=None):
        """`rule` None picks by row count as the reference's op does (int8_linear.py:92-98); 'decode' applies
        the decode kernel's per-row formula to every row (what that many single-row calls compute)."""
        if self.q is None:
            return x @ self.weight.t()
        if self._qf is None:
            self._qf = self.q.float()  # exact image of the codes, cached
        if x.dtype != torch.bfloat16:
            return (x.float() @ self._qf.t() * self.s).to(x.dtype)
        if rule == 'decode' or (rule is None and x.reshape(-1, x.shape[-1]).shape[0] <= MAX_DECODE_ROWS):
            return (self._sum(x) * self.s).to(torch.bfloat16)
        acc = x.float() @ self._qf.t()  # prefill: the library GEMM, no split-K form
        return (acc.to(torch.bfloat16).float() * self.s).to(torch.bfloat16)


class Qwen3Oracle:
    """Batch-1 Qwen3 forward over a static KV cache of `cap` slots."""

    def __init__(self, shape, weights, dtype=torch.bfloat16, cap=256, inv_freq=None):
        self.shape, self.dtype, self.cap = shape, dtype, cap
        w = {k: v.cpu() for k, v in weights.items()}
        cvt = (lambda t: t.to(dtype))

        def lin(name):
            if name + '.qweight' in w:
                return Linear(qweight=w[name + '.qweight'], scale=w[name + '.scale'].float())
            return Linear(weight=cvt(w[name + '.weight']))

        self.embed = cvt(w['model.embed_tokens.weight'])
        self.layers = []
        for i in range(shape.layers):
            p = f'model.layers.{i}.'
            layer = {n: lin(p + n) for n in LINEARS}
            for n in ('input_layernorm', 'post_attention_layernorm', 'self_attn.q_norm', 'self_attn.k_norm'):
                layer[n] = cvt(w[p + n + '.weight'])
            self.layers.append(layer)
        self.norm = cvt(w['model.norm.weight'])
        if 'lm_head.qweight' in w or 'lm_head.weight' in w:
            self.lm_head = lin('lm_head')
        else:  # tied head on the embedding
            self.lm_head = Linear(weight=self.embed)
        self.cos, self.sin = rope_tables(shape, cap, dtype, inv_freq)
        self.reset()

    def set_ksplit(self, ksplit):
        """Sum every int8 linear's decode formula in `ksplit` chunks (Linear.ksplit); 1 is the one-pass form."""
        for layer in self.layers:
            for n in LINEARS:
                layer[n].ksplit = ksplit
        self.lm_head.ksplit = ksplit

    def reset(self):
        s = self.shape
        self.k_cache = [torch.zeros(s.kv_heads, self.cap, s.head_dim, dtype=self.dtype) for _ in range(s.layers)]
        self.v_cache = [torch.zeros(s.kv_heads, self.cap, s.head_dim, dtype=self.dtype) for _ in range(s.layers)]

    def _attention(self, q, layer, pos0, chunk=512):
        """q [T, Hq, D] at positions pos0..pos0+T-1 over cache slots 0..position: fp32 math.

        Query rows are taken `chunk` at a time (each row's result depends on that row alone), so a long prompt
        never holds more than Hq x chunk x slots scores."""
        s = self.shape
        t = q.shape[0]
        g = s.heads // s.kv_heads
        n = pos0 + t
        k = self.k_cache[layer][:, :n].float()
        v = self.v_cache[layer][:, :n].float()
        k = k.repeat_interleave(g, dim=0)  # [Hq, n, D]
        v = v.repeat_interleave(g, dim=0)
        kt = k.transpose(1, 2)
        slots = torch.arange(n)
        out = torch.empty(t, s.heads * s.head_dim, dtype=self.dtype)
        for r0 in range(0, t, chunk):
            r1 = min(t, r0 + chunk)
            m = n - (t - r1)  # slots the last row of this chunk may see
            qf = q[r0:r1].float().transpose(0, 1)  # [Hq, rows, D]
            scores = (qf @ kt[:, :, :m]) * (s.head_dim ** -0.5)
            allowed = slots[None, :m] <= (pos0 + torch.arange(r0, r1))[:, None]
            scores = scores.masked_fill(~allowed[None], float('-inf'))
            o = torch.softmax(scores, dim=-1) @ v[:, :m]  # [Hq, rows, D]
            out[r0:r1] = o.transpose(0, 1).reshape(r1 - r0, s.heads * s.head_dim).to(self.dtype)
        return out

    @torch.no_grad()
    def forward(self, tokens, pos0, all_logits=False, rule=None):
        """tokens: 1-D ids at positions pos0.. ; writes the cache; returns last-row logits [vocab].

        all_logits: return every row's logits [T, vocab] instead. rule='decode': every linear uses the decode
        formula on every row, so T rows at once compute what T single-token decode steps would (each row sees
        slots 0..its own position): the teacher-forced form of a greedy decode."""
        s = self.shape
        tokens = torch.as_tensor(tokens, dtype=torch.long).reshape(-1)
        t = tokens.numel()
        if pos0 + t > self.cap:
            raise ValueError('oracle cache capacity exceeded')
        x = self.embed[tokens]  # [T, H]
        cos = self.cos[pos0:pos0 + t][:, None, :]
        sin = self.sin[pos0:pos0 + t][:, None, :]
        for i, L in enumerate(self.layers):
            h = rms_norm(x, L['input_layernorm'], s.rms_eps)
            q = L['self_attn.q_proj'](h, rule).view(t, s.heads, s.head_dim)
            k = L['self_attn.k_proj'](h, rule).view(t, s.kv_heads, s.head_dim)
            v = L['self_attn.v_proj'](h, rule).view(t, s.kv_heads, s.head_dim)
            q = rms_norm(q, L['self_attn.q_norm'], s.rms_eps)
            k = rms_norm(k, L['self_attn.k_norm'], s.rms_eps)
            q = (q * cos) + (rotate_half(q) * sin)
            k = (k * cos) + (rotate_half(k) * sin)
            self.k_cache[i][:, pos0:pos0 + t] = k.transpose(0, 1)
            self.v_cache[i][:, pos0:pos0 + t] = v.transpose(0, 1)
            a = self._attention(q, i, pos0)
            x = x + L['self_attn.o_proj'](a, rule)
            h = rms_norm(x, L['post_attention_layernorm'], s.rms_eps)
            x = x + L['mlp.down_proj'](F.silu(L['mlp.gate_proj'](h, rule)) * L['mlp.up_proj'](h, rule), rule)
        # the head always sees one row per call in a decode (logits_to_keep=1): the decode formula
        if all_logits:
            return self.lm_head(rms_norm(x, self.norm, s.rms_eps), 'decode')
        x = rms_norm(x[-1:], self.norm, s.rms_eps)
        return self.lm_head(x, 'decode')[0]

    def greedy(self, prompt, n_new, with_margins=False):
        """Greedy ids of n_new tokens after `prompt` (and each step's top-1 minus top-2 logit if asked)."""
        self.reset()
        prompt = torch.as_tensor(prompt, dtype=torch.long).reshape(-1)
        logits = self.forward(prompt, 0)
        out, margins = [], []
        pos = prompt.numel()
        for i in range(n_new):
            top = logits.float().topk(2).values
            margins.append(float(top[0] - top[1]))
            tok = int(torch.argmax(logits))
            out.append(tok)
            if i + 1 < n_new:
                logits = self.forward([tok], pos)
                pos += 1
        return (out, margins) if with_margins else out


def random_weights(shape, seed=0, std=0.02, norm_jitter=0.0, dtype=torch.bfloat16):
    """Seeded random-init weights with transformers' names: N(0, std) linears and embedding, norms 1 (+ jitter)."""
    g = torch.Generator().manual_seed(seed)
    s = shape
    w = {'model.embed_tokens.weight': (torch.randn(s.vocab, s.hidden, generator=g) * std).to(dtype)}
    dims = {'self_attn.q_proj': (s.heads * s.head_dim, s.hidden), 'self_attn.k_proj': (s.kv_heads * s.head_dim, s.hidden),
            'self_attn.v_proj': (s.kv_heads * s.head_dim, s.hidden), 'self_attn.o_proj': (s.hidden, s.heads * s.head_dim),
            'mlp.gate_proj': (s.inter, s.hidden), 'mlp.up_proj': (s.inter, s.hidden), 'mlp.down_proj': (s.hidden, s.inter)}

    def norm(n):
        return (1.0 + norm_jitter * torch.randn(n, generator=g)).to(dtype)

    for i in range(s.layers):
        p = f'model.layers.{i}.'
        for name, (n, k) in dims.items():
            w[p + name + '.weight'] = (torch.randn(n, k, generator=g) * std).to(dtype)
        w[p + 'input_layernorm.weight'] = norm(s.hidden)
        w[p + 'post_attention_layernorm.weight'] = norm(s.hidden)
        w[p + 'self_attn.q_norm.weight'] = norm(s.head_dim)
        w[p + 'self_attn.k_norm.weight'] = norm(s.head_dim)
    w['model.norm.weight'] = norm(s.hidden)
    if not s.tied:
        w['lm_head.weight'] = (torch.randn(s.vocab, s.hidden, generator=g) * std).to(dtype)
    return w


def quantize_weights(weights, shape):
    """Replace every linear (and the head; a tied head is quantised from the embedding) by qweight/scale."""
    out = {}
    for k, v in weights.items():
        base = k[:-len('.weight')] if k.endswith('.weight') else None
        if base and (base.endswith(LINEARS) or base == 'lm_head'):
            out[base + '.qweight'], out[base + '.scale'] = quantize_rows(v)
        else:
            out[k] = v
    if 'lm_head.qweight' not in out:
        out['lm_head.qweight'], out['lm_head.scale'] = quantize_rows(weights['model.embed_tokens.weight'])
    return out
