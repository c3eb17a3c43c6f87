"""Batch-1 Qwen3 int8 decode engine on the gfx950 kernels.

The decode step of a Qwen3 decoder (transformers' models/qwen3/modeling_qwen3.py),
every linear int8 weight-only, run entirely through libegpt_hip.so and captured as
one graph: the host launches nothing per token but the graph replay. It is the
MI355X counterpart of the reference's captured step (research/realmodel/fast_decode.py:
GraphGreedyDecoder._step / _capture, :45-64) with the Inductor-compiled HF forward
replaced by explicit kernels.

Data layout in HBM (per layer, all device-resident for the life of the engine):
  qkv_q   int8 [(Hq + 2 Hkv) * D, hidden]   q, k, v projections stacked by rows
  qkv_s   fp32 [(Hq + 2 Hkv) * D]           their per-row scales (rows are independent,
                                            so stacking is bit-identical to 3 GEMVs)
  o_q     int8 [hidden, Hq * D]             o_proj
  gu_q    int8 [2 * inter, hidden]          gate rows then up rows
  down_q  int8 [hidden, inter]
  k_cache, v_cache  bf16 [layers, Hkv, cap, D]  static cache, slot = position
plus the bf16 embedding [vocab, hidden], the int8 lm_head (a tied head is an int8
copy of the embedding, research/realmodel/int8_linear.py:154-155) and bf16 RoPE
tables [cap, D] built with transformers' formula.

Step (token t at position p; writes K/V slot p, attends to slots 0..p):
  embed -> [add+]RMSNorm -> QKV GEMV -> q/k norm + RoPE + cache write -> split-K
  attention + combine -> o GEMV -> add+RMSNorm -> gate_up GEMV -> SiLU*up ->
  down GEMV -> ... -> add+final RMSNorm -> lm_head GEMV -> argmax (token, p + 1).
Prefill runs the same kernels over all prompt rows, outside the graph; linears past 16
rows take the reference's prefill formula (int8_linear.py:96-97) on the MFMA GEMM that
reads the int8 weights, and long prompts (use_prompt_kernel) the causal MFMA prefill
attention (egpt_prefill_attn).
"""

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .int8_linear import MAX_DECODE_ROWS, int8_gemm, quantize_weight

# Prompt attention runs either the causal prompt-attention kernel (egpt_prefill_attn: one pass over the prefix per
# block of queries) or the split-K decode kernel with the prompt's query rows as batch rows (each row rescans its own
# prefix). Measured on the MI355X at fresh prompts (16 / 8 and 32 / 8 heads, D 128, 20 calls per graph): the decode
# kernel 4.2-10.2 us against 6.7-13.2 us for the prompt kernel at 32-128 rows, about equal at 192, slower at 256 (the
# prompt kernel's few blocks are latency-bound on short prompts). The decode kernel's cost grows with rows x prefix,
# so it takes prompts of at most PREFILL_KERNEL_MAX_ROWS rows anywhere, and longer ones only while their last
# position stays below DECODE_KERNEL_MAX_CONTEXT.
PREFILL_KERNEL_MAX_ROWS = 64
DECODE_KERNEL_MAX_CONTEXT = 160


def use_prompt_kernel(rows, pos0):
    """Whether `rows` query rows at positions pos0 .. pos0 + rows - 1 take egpt_prefill_attn."""
    return rows > PREFILL_KERNEL_MAX_ROWS and pos0 + rows > DECODE_KERNEL_MAX_CONTEXT

# Head geometry the decode-step attention kernels take (egpt_qwen3_decode_step, egpt_decode_attn).
SUPPORTED_HEAD_DIMS = (32, 64, 128)
SUPPORTED_GROUPS = (1, 2, 4, 8)

LINEARS = ('self_attn.q_proj', 'self_attn.k_proj', 'self_attn.v_proj', 'self_attn.o_proj',
           'mlp.gate_proj', 'mlp.up_proj', 'mlp.down_proj')


@dataclass(frozen=True)
class Qwen3Config:
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

    @classmethod
    def from_hf(cls, cfg):
        rope = getattr(cfg, 'rope_parameters', None) or {}
        theta = rope.get('rope_theta', getattr(cfg, 'rope_theta', 1e6))
        head_dim = getattr(cfg, 'head_dim', None) or cfg.hidden_size // cfg.num_attention_heads
        return cls(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
                   cfg.num_attention_heads, cfg.num_key_value_heads, head_dim, float(theta), cfg.rms_norm_eps,
                   bool(getattr(cfg, 'tie_word_embeddings', False)))

    def weight_bytes(self):
        """int8 linear bytes + fp32 scales streamed per decode step (lm_head included)."""
        d = self.head_dim
        per_layer_rows = (self.heads + 2 * self.kv_heads) * d + self.hidden + 2 * self.inter + self.hidden
        per_layer = ((self.heads + 2 * self.kv_heads) * d * self.hidden + self.hidden * self.heads * d
                     + 2 * self.inter * self.hidden + self.hidden * self.inter)
        return (self.layers * per_layer + self.vocab * self.hidden,
                4 * (self.layers * per_layer_rows + self.vocab))

    def kv_bytes_per_slot(self):
        return self.layers * self.kv_heads * self.head_dim * 2 * 2


QWEN3_1_7B = Qwen3Config(vocab=151936, hidden=2048, inter=6144, layers=28, heads=16, kv_heads=8, head_dim=128)
QWEN3_8B = Qwen3Config(vocab=151936, hidden=4096, inter=12288, layers=36, heads=32, kv_heads=8, head_dim=128,
                       tied=False)


def rope_tables(cfg, length, inv_freq=None):
    """bf16 cos/sin [length, head_dim] with transformers' arithmetic (fp32 products, cos/sin, cast).

    Built once on the host at engine construction; `inv_freq` overrides the fp32
    formula (a transformers model cast with .to(bfloat16) carries a bf16 copy).
    """
    d = cfg.head_dim
    if inv_freq is None:
        inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    inv_freq = inv_freq.detach().cpu().float()
    pos = torch.arange(length, dtype=torch.float)
    freqs = (inv_freq[None, :, None] @ pos[None, None, :]).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _as_int8(weights, name):
    """(qweight, scale) of linear `name`, quantising a float weight if that is what is given."""
    if name + '.qweight' in weights:
        return weights[name + '.qweight'], weights[name + '.scale'].float()
    return quantize_weight(weights[name + '.weight'])


def pack_qwen3(cfg, weights):
    """The engine's packed int8 layout from transformers-named weights, on the device they are on.

    Returns {'layers': [{'qkv_q', 'qkv_s', 'o_q', 'o_s', 'gu_q', 'gu_s', 'down_q', 'down_s', 'in_w', 'post_w',
    'qn_w', 'kn_w'}, ...], 'embed', 'norm_w', 'head_q', 'head_s'}: linears given as `<name>.qweight` /
    `<name>.scale` are taken as they are, float `<name>.weight` ones are quantised
    (research/realmodel/int8_linear.py:106-117); a tied head is an int8 copy of the embedding
    (int8_linear.py:154-155) and the embedding stays bf16.
    """
    bf = torch.bfloat16
    layers = []
    for i in range(cfg.layers):
        p = f'model.layers.{i}.'
        qs = [_as_int8(weights, p + n) for n in LINEARS]
        layers.append({
            'qkv_q': torch.cat([qs[0][0], qs[1][0], qs[2][0]]),
            'qkv_s': torch.cat([qs[0][1], qs[1][1], qs[2][1]]).float(),
            'o_q': qs[3][0], 'o_s': qs[3][1].float(),
            'gu_q': torch.cat([qs[4][0], qs[5][0]]),
            'gu_s': torch.cat([qs[4][1], qs[5][1]]).float(),
            'down_q': qs[6][0], 'down_s': qs[6][1].float(),
            'in_w': weights[p + 'input_layernorm.weight'].to(bf),
            'post_w': weights[p + 'post_attention_layernorm.weight'].to(bf),
            'qn_w': weights[p + 'self_attn.q_norm.weight'].to(bf),
            'kn_w': weights[p + 'self_attn.k_norm.weight'].to(bf),
        })
        del qs
    embed = weights['model.embed_tokens.weight'].to(bf)
    if 'lm_head.qweight' in weights or 'lm_head.weight' in weights:
        hq, hs = _as_int8(weights, 'lm_head')
    else:
        hq, hs = quantize_weight(embed)
    return {'layers': layers, 'embed': embed, 'norm_w': weights['model.norm.weight'].to(bf),
            'head_q': hq, 'head_s': hs.float()}


def _expect(what, t, dtype, shape):
    if t.dtype != dtype or tuple(t.shape) != tuple(shape):
        raise ValueError(f'{what}: {t.dtype} {tuple(t.shape)}, expected {dtype} {tuple(shape)}')


def check_packed(cfg, packed):
    """Every tensor of the packed layout (pack_qwen3's result, or a checkpoint's) against the config, dtype and
    shape: weights that do not match fail here (ValueError), not in a kernel that would read past the end of a
    short tensor."""
    d, hq, hkv = cfg.head_dim, cfg.heads, cfg.kv_heads
    want = {'qkv_q': ((hq + 2 * hkv) * d, cfg.hidden), 'o_q': (cfg.hidden, hq * d), 'gu_q': (2 * cfg.inter, cfg.hidden),
            'down_q': (cfg.hidden, cfg.inter)}
    norms = {'in_w': cfg.hidden, 'post_w': cfg.hidden, 'qn_w': d, 'kn_w': d}
    if len(packed['layers']) != cfg.layers:
        raise ValueError(f'{len(packed["layers"])} layers given, the config has {cfg.layers}')
    for i, L in enumerate(packed['layers']):
        for key, shape in want.items():
            _expect(f'layer {i} {key}', L[key], torch.int8, shape)
            _expect(f'layer {i} {key[:-1]}s', L[key[:-1] + 's'], torch.float32, (shape[0],))
        for key, n in norms.items():
            _expect(f'layer {i} {key}', L[key], torch.bfloat16, (n,))
    _expect('embed', packed['embed'], torch.bfloat16, (cfg.vocab, cfg.hidden))
    _expect('final_norm', packed['norm_w'], torch.bfloat16, (cfg.hidden,))
    _expect('lm_head qweight', packed['head_q'], torch.int8, (cfg.vocab, cfg.hidden))
    _expect('lm_head scale', packed['head_s'], torch.float32, (cfg.vocab,))


class Qwen3Int8Engine:
    """Static-cache batch-1 Qwen3 decoder with int8 linears; one graph replay per token.

    `weights` holds transformers-named tensors (see pack_qwen3), or, with `packed=True`,
    the packed layout pack_qwen3 returns (what efficientgpt_amd.checkpoint stores).
    """

    def __init__(self, cfg, weights, max_cache_len, device='cuda', inv_freq=None, packed=False):
        if max_cache_len < 1:
            raise ValueError('max_cache_len must be >= 1')
        if cfg.head_dim not in SUPPORTED_HEAD_DIMS or cfg.heads % cfg.kv_heads or \
                cfg.heads // cfg.kv_heads not in SUPPORTED_GROUPS:
            raise ValueError(f'head_dim {cfg.head_dim} with {cfg.heads} / {cfg.kv_heads} heads: the attention kernels '
                             f'take head dims {SUPPORTED_HEAD_DIMS} and {SUPPORTED_GROUPS} query heads per kv head')
        self.cfg = cfg
        self.device = torch.device(device)
        dev, bf = self.device, torch.bfloat16
        c = cfg
        self.n_qkv = (c.heads + 2 * c.kv_heads) * c.head_dim

        def put(t, dtype=None):
            return t.to(device=dev, dtype=dtype or t.dtype).contiguous()

        # Prompt passes fold the residual add + RMSNorm after o_proj and down_proj into the split-K GEMM's reduce
        # (egpt_int8_gemm_add_rmsnorm), q/k norm + RoPE into the split-K QKV reduce (egpt_int8_gemm_qk_norm_rope),
        # the next layer's input norm into the down projection and SwiGLU into the gate/up GEMM
        # (egpt_int8_gemm_swiglu); False runs the separate linear, egpt_add_rmsnorm, egpt_qk_norm_rope and
        # egpt_silu_mul calls instead (the same bits).
        self.fold_norms = True
        pk = weights if packed else pack_qwen3(c, weights)
        check_packed(c, pk)
        self.layers = [{k: put(v) for k, v in L.items()} for L in pk['layers']]
        self.embed = put(pk['embed'], bf)
        self.norm_w = put(pk['norm_w'], bf)
        self.head_q, self.head_s = put(pk['head_q']), put(pk['head_s'], torch.float32)
        self.inv_freq = None if inv_freq is None else inv_freq.detach().float().cpu()
        del pk
        self._init_state(int(max_cache_len))

    def _init_state(self, cap):
        """Everything that depends on the cache capacity: RoPE tables, the K/V cache, the token / position state,
        activation rows, workspaces and the fused step's descriptor. The weights are not touched."""
        c, dev, bf = self.cfg, self.device, torch.bfloat16
        d = c.head_dim
        self.cap = cap
        cos, sin = rope_tables(c, cap, self.inv_freq)
        self.cos, self.sin = cos.to(dev).contiguous(), sin.to(dev).contiguous()

        # static state and activations
        self.k_cache = torch.zeros(c.layers, c.kv_heads, cap, d, device=dev, dtype=bf)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.token = torch.zeros(1, dtype=torch.long, device=dev)
        self.position = torch.zeros(1, dtype=torch.long, device=dev)
        self.x = torch.zeros(1, c.hidden, device=dev, dtype=bf)
        self.h = torch.zeros(1, c.hidden, device=dev, dtype=bf)
        self.qkv = torch.zeros(1, self.n_qkv, device=dev, dtype=bf)
        self.qrot = torch.zeros(1, c.heads * d, device=dev, dtype=bf)
        self.attn = torch.zeros(1, c.heads * d, device=dev, dtype=bf)
        self.o = torch.zeros(1, c.hidden, device=dev, dtype=bf)
        self.gu = torch.zeros(1, 2 * c.inter, device=dev, dtype=bf)
        self.act = torch.zeros(1, c.inter, device=dev, dtype=bf)
        self.down = torch.zeros(1, c.hidden, device=dev, dtype=bf)
        self.logits = torch.zeros(1, c.vocab, device=dev, dtype=bf)
        # every step's token, stored by the step itself at slot (new position % cap) of pinned host memory
        self.token_ring = torch.full((cap,), -1, dtype=torch.long, pin_memory=True)
        self._ring_dev = _lib.host_device_pointer(self.token_ring.data_ptr())
        lib = _lib.lib()
        self.nsplit = lib.egpt_qwen3_step_default_splits(c.heads, c.kv_heads, d, cap)
        need = ctypes.c_size_t()
        _lib.check('egpt_decode_attn_workspace',
                   lib.egpt_decode_attn_workspace(1, c.heads, c.kv_heads, cap, d, self.nsplit, need))
        self.attn_ws = torch.zeros(need.value, device=dev, dtype=torch.uint8)
        _lib.check('egpt_argmax_workspace', lib.egpt_argmax_workspace(c.vocab, need))
        self.arg_ws = torch.zeros(need.value, device=dev, dtype=torch.uint8)
        self._build_step_desc()
        self.graph = None

    def with_capacity(self, max_cache_len):
        """An engine over the same weight tensors (shared, not copied) with its own cache of max_cache_len slots,
        its own state and its own graph: one per capacity bucket of a decoder pool."""
        if max_cache_len < 1:
            raise ValueError('max_cache_len must be >= 1')
        other = object.__new__(type(self))
        other.cfg, other.device, other.n_qkv = self.cfg, self.device, self.n_qkv
        other.layers, other.embed, other.norm_w = self.layers, self.embed, self.norm_w
        other.head_q, other.head_s, other.inv_freq = self.head_q, self.head_s, self.inv_freq
        other.fold_norms = self.fold_norms
        if hasattr(self, 'weights'):
            other.weights = self.weights
        other._init_state(int(max_cache_len))
        return other

    def _build_step_desc(self):
        """The egpt_qwen3_step descriptor of the fused decode step (pointers into this engine's tensors)."""
        c, lib = self.cfg, _lib.lib()
        ptr = (lambda t: t.data_ptr())
        self._layers_c = (_lib.Qwen3Layer * c.layers)()
        for i, L in enumerate(self.layers):
            e = self._layers_c[i]
            e.qkv_w, e.qkv_s = ptr(L['qkv_q']), ptr(L['qkv_s'])
            e.o_w, e.o_s = ptr(L['o_q']), ptr(L['o_s'])
            e.gu_w, e.gu_s = ptr(L['gu_q']), ptr(L['gu_s'])
            e.down_w, e.down_s = ptr(L['down_q']), ptr(L['down_s'])
            e.in_norm, e.post_norm = ptr(L['in_w']), ptr(L['post_w'])
            e.q_norm, e.k_norm = ptr(L['qn_w']), ptr(L['kn_w'])
            e.k_cache, e.v_cache = ptr(self.k_cache[i]), ptr(self.v_cache[i])
        d = _lib.Qwen3Step()
        d.layers, d.hidden, d.inter = c.layers, c.hidden, c.inter
        d.heads, d.kv_heads, d.head_dim, d.vocab = c.heads, c.kv_heads, c.head_dim, c.vocab
        d.cap, d.nsplit, d.eps = self.cap, self.nsplit, c.rms_eps
        d.layer = ctypes.cast(self._layers_c, ctypes.c_void_p)
        d.embed, d.final_norm = ptr(self.embed), ptr(self.norm_w)
        d.head_w, d.head_s = ptr(self.head_q), ptr(self.head_s)
        d.rope_cos, d.rope_sin = ptr(self.cos), ptr(self.sin)
        d.token, d.position = ptr(self.token), ptr(self.position)
        d.x, d.qkv, d.attn, d.act, d.logits = ptr(self.x), ptr(self.qkv), ptr(self.attn), ptr(self.act), ptr(self.logits)
        need = ctypes.c_size_t()
        _lib.check('egpt_qwen3_step_workspace', lib.egpt_qwen3_step_workspace(ctypes.byref(d), ctypes.byref(need)))
        # attention partials and argmax partials: every step writes them before it reads them
        self.step_ws = torch.empty(need.value, device=self.device, dtype=torch.uint8)
        d.workspace, d.workspace_bytes = ptr(self.step_ws), need.value
        if self._ring_dev:
            d.token_ring, d.token_ring_slots = self._ring_dev, self.cap
        self._step_c = d

    # ------------------------------------------------------------------ construction helpers

    @classmethod
    def from_int8(cls, path, max_cache_len, device='cuda'):
        """Engine over an efficientgpt_amd.checkpoint file: the stored int8 layout, no re-quantisation."""
        from .checkpoint import load_int8
        cfg, packed, inv_freq = load_int8(path)
        return cls(cfg, packed, max_cache_len, device=device, inv_freq=inv_freq, packed=True)

    @classmethod
    @torch.no_grad()
    def random(cls, cfg, max_cache_len, seed=0, std=0.02, device='cuda', keep_weights=False):
        """Random-init weights N(0, std) (bf16, norms 1), quantised per output channel on the device.

        keep_weights: also keep a HOST copy of the transformers-named int8 weights as `.weights` (what a CPU
        model of the same network is built from); the device holds only the engine's packed layout."""
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)

        def randn(n, k):
            return (torch.randn(n, k, generator=g, device=dev) * std).to(torch.bfloat16)

        c = cfg
        d = c.head_dim
        dims = {'self_attn.q_proj': (c.heads * d, c.hidden), 'self_attn.k_proj': (c.kv_heads * d, c.hidden),
                'self_attn.v_proj': (c.kv_heads * d, c.hidden), 'self_attn.o_proj': (c.hidden, c.heads * d),
                'mlp.gate_proj': (c.inter, c.hidden), 'mlp.up_proj': (c.inter, c.hidden),
                'mlp.down_proj': (c.hidden, c.inter)}
        w = {'model.embed_tokens.weight': randn(c.vocab, c.hidden)}
        ones = torch.ones(c.hidden, device=dev, dtype=torch.bfloat16)
        ones_d = torch.ones(d, device=dev, dtype=torch.bfloat16)
        for i in range(c.layers):
            p = f'model.layers.{i}.'
            for name, (n, k) in dims.items():
                w[p + name + '.qweight'], w[p + name + '.scale'] = quantize_weight(randn(n, k))
            w[p + 'input_layernorm.weight'] = ones
            w[p + 'post_attention_layernorm.weight'] = ones
            w[p + 'self_attn.q_norm.weight'] = ones_d
            w[p + 'self_attn.k_norm.weight'] = ones_d
        w['model.norm.weight'] = ones
        if not c.tied:
            w['lm_head.qweight'], w['lm_head.scale'] = quantize_weight(randn(c.vocab, c.hidden))
        else:
            w['lm_head.qweight'], w['lm_head.scale'] = quantize_weight(w['model.embed_tokens.weight'])
        eng = cls(cfg, w, max_cache_len, device=dev)
        if keep_weights:
            eng.weights = {k: v.cpu() for k, v in w.items()}
        del w
        return eng

    @classmethod
    @torch.no_grad()
    def from_hf(cls, model, max_cache_len, quantize=False):
        """Engine over a transformers Qwen3ForCausalLM whose linears (lm_head included) are int8, as
        `quantize_model(model)` leaves them; their codes and scales are taken as they are.

        A model with float linears is refused (ValueError) unless `quantize=True`: the engine runs every
        linear on the int8 contract, so running such a model here would change its output. With
        quantize=True the float linears are quantised per output channel (research/realmodel/int8_linear.py:
        106-117) and a tied float head from the embedding."""
        cfg = Qwen3Config.from_hf(model.config)
        sd = dict(model.state_dict())
        names = [f'model.layers.{i}.{n}' for i in range(cfg.layers) for n in LINEARS] + ['lm_head']
        floats = [n for n in names if n + '.qweight' not in sd]
        if floats and not quantize:
            raise ValueError(f'{len(floats)} linear layers are not int8 (first: {floats[0]}); this decoder runs the '
                             'int8 weight-only path: call quantize_model(model) first, or pass quantize=True')
        if 'lm_head.qweight' not in sd and cfg.tied:
            sd.pop('lm_head.weight', None)  # tied float head: quantise from the embedding
        device = next(model.parameters()).device
        return cls(cfg, sd, max_cache_len, device=device, inv_freq=model.model.rotary_emb.inv_freq)

    # ------------------------------------------------------------------ kernels

    def _stream(self):
        return _lib.stream_ptr(self.device)

    def _prefill_workspace(self, rows):
        """One split-K workspace for a prompt pass of `rows` rows: the largest any of the layer's linears (and
        their fused reduce) needs at that row count, allocated once per pass and shared by every GEMM of it
        (the calls run in stream order, so none overlaps another)."""
        lib, c = _lib.lib(), self.cfg
        d = c.head_dim
        need, most = ctypes.c_size_t(), 0
        for n, k in ((self.n_qkv, c.hidden), (c.hidden, c.heads * d), (2 * c.inter, c.hidden), (c.hidden, c.inter)):
            _lib.check('egpt_int8_gemm_workspace', lib.egpt_int8_gemm_workspace(rows, n, k, ctypes.byref(need)))
            most = max(most, need.value)
        return torch.empty(most, device=self.device, dtype=torch.uint8) if most else None

    def _linear(self, x, q, s, out, rows, ws=None):
        """out[:rows] = int8 linear of x[:rows]; the reference's row rule (<= 16 rows: GEMV kernel, more: the
        prefill GEMM, splitting K through `ws` when given)."""
        if rows <= MAX_DECODE_ROWS:
            _lib.check('egpt_int8_gemv', _lib.lib().egpt_int8_gemv(
                x.data_ptr(), x.stride(0), q.data_ptr(), q.stride(0), s.data_ptr(), out.data_ptr(), out.stride(0),
                rows, q.shape[0], q.shape[1], self._stream()))
        else:
            int8_gemm(x[:rows], q, s, out=out[:rows], workspace=ws)

    def _linear_add_norm(self, xin, q, s, out, x, norm_w, h, rows, ws=None):
        """x = bf16(x + linear(xin)) and h = RMSNorm(x) * norm_w for `rows` rows. Split-K shapes take
        egpt_int8_gemm_add_rmsnorm (one launch after the split slices instead of the reduce and the norm, the
        same bits); the others, or every shape when `fold_norms` is off, the linear into `out`, then
        egpt_add_rmsnorm."""
        lib, c, st = _lib.lib(), self.cfg, self._stream()
        if rows > MAX_DECODE_ROWS and self.fold_norms:
            need = ctypes.c_size_t()
            _lib.check('egpt_int8_gemm_workspace',
                       lib.egpt_int8_gemm_workspace(rows, q.shape[0], q.shape[1], ctypes.byref(need)))
            if need.value:
                if ws is None or ws.numel() < need.value:
                    ws = torch.empty(need.value, device=self.device, dtype=torch.uint8)
                r = lib.egpt_int8_gemm_add_rmsnorm(xin.data_ptr(), xin.stride(0), q.data_ptr(), q.stride(0),
                                                   s.data_ptr(), x.data_ptr(), x.stride(0), norm_w.data_ptr(),
                                                   h.data_ptr(), h.stride(0), rows, q.shape[0], q.shape[1], c.rms_eps,
                                                   ws.data_ptr(), ws.numel(), st)
                if r != _lib.EGPT_ERR_UNSUPPORTED:
                    _lib.check('egpt_int8_gemm_add_rmsnorm', r)
                    return
        self._linear(xin, q, s, out, rows, ws)
        _lib.check('egpt_add_rmsnorm', lib.egpt_add_rmsnorm(x.data_ptr(), x.stride(0), out.data_ptr(), out.stride(0),
                                                            norm_w.data_ptr(), h.data_ptr(), h.stride(0), rows,
                                                            c.hidden, c.rms_eps, st))

    def _layer(self, i, rows, x, h, qkv, qrot, attn, o, gu, act, down, positions, pos_stride, first, pos0=0,
               normed=False, ws=None):
        """One layer over `rows` rows. `normed`: h already holds the layer's input RMSNorm (the previous layer's
        down projection folded it in); the layer then folds the next layer's input norm into its own down
        projection when there is a next layer (returns True), and leaves x + down to the caller otherwise. `ws`:
        the pass's split-K workspace (_prefill_workspace)."""
        lib, c, L, st = _lib.lib(), self.cfg, self.layers[i], self._stream()
        d = c.head_dim
        if normed:
            pass
        elif first:
            _lib.check('egpt_rmsnorm', lib.egpt_rmsnorm(x.data_ptr(), x.stride(0), L['in_w'].data_ptr(), h.data_ptr(),
                                                        h.stride(0), rows, c.hidden, c.rms_eps, st))
        else:
            _lib.check('egpt_add_rmsnorm', lib.egpt_add_rmsnorm(
                x.data_ptr(), x.stride(0), down.data_ptr(), down.stride(0), L['in_w'].data_ptr(), h.data_ptr(),
                h.stride(0), rows, c.hidden, c.rms_eps, st))
        kc, vc = self.k_cache[i], self.v_cache[i]
        fused = _lib.EGPT_ERR_UNSUPPORTED
        if rows > MAX_DECODE_ROWS and self.fold_norms and ws is not None:
            # split-K QKV: the reduce, q/k norm, RoPE and cache write in one launch after the split slices
            fused = lib.egpt_int8_gemm_qk_norm_rope(
                h.data_ptr(), h.stride(0), L['qkv_q'].data_ptr(), L['qkv_q'].stride(0), L['qkv_s'].data_ptr(),
                positions.data_ptr(), L['qn_w'].data_ptr(), L['kn_w'].data_ptr(), self.cos.data_ptr(),
                self.sin.data_ptr(), qrot.data_ptr(), qrot.stride(0), kc.data_ptr(), vc.data_ptr(), kc.stride(0),
                kc.stride(1), rows, c.heads, c.kv_heads, d, c.hidden, self.cap, c.rms_eps, ws.data_ptr(), ws.numel(),
                st)
        if fused == _lib.EGPT_ERR_UNSUPPORTED:
            self._linear(h, L['qkv_q'], L['qkv_s'], qkv, rows, ws)
            _lib.check('egpt_qk_norm_rope', lib.egpt_qk_norm_rope(
                qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), L['qn_w'].data_ptr(), L['kn_w'].data_ptr(),
                self.cos.data_ptr(), self.sin.data_ptr(), qrot.data_ptr(), qrot.stride(0), kc.data_ptr(),
                vc.data_ptr(), kc.stride(0), kc.stride(1), rows, c.heads, c.kv_heads, d, self.cap, c.rms_eps, st))
        else:
            _lib.check('egpt_int8_gemm_qk_norm_rope', fused)
        if use_prompt_kernel(rows, pos0):
            _lib.check('egpt_prefill_attn', lib.egpt_prefill_attn(
                qrot.data_ptr(), qrot.stride(0), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                attn.data_ptr(), attn.stride(0), rows, c.heads, c.kv_heads, d, self.cap, pos0, d ** -0.5, st))
        else:
            self._kernel_attention(qrot, kc, vc, rows, positions, pos_stride, attn)
        self._linear_add_norm(attn, L['o_q'], L['o_s'], o, x, L['post_w'], h, rows, ws)
        fused = _lib.EGPT_ERR_UNSUPPORTED
        if rows > MAX_DECODE_ROWS and self.fold_norms:  # SwiGLU in the gate/up GEMM's epilogue
            fused = lib.egpt_int8_gemm_swiglu(h.data_ptr(), h.stride(0), L['gu_q'].data_ptr(), L['gu_q'].stride(0),
                                              L['gu_s'].data_ptr(), act.data_ptr(), act.stride(0), rows, c.inter,
                                              c.hidden, st)
        if fused == _lib.EGPT_ERR_UNSUPPORTED:
            self._linear(h, L['gu_q'], L['gu_s'], gu, rows, ws)
            _lib.check('egpt_silu_mul', lib.egpt_silu_mul(gu.data_ptr(), gu.stride(0), c.inter, act.data_ptr(),
                                                          act.stride(0), rows, st))
        else:
            _lib.check('egpt_int8_gemm_swiglu', fused)
        if i + 1 < c.layers and rows > MAX_DECODE_ROWS and self.fold_norms:
            # the next layer's input norm folds into this projection
            self._linear_add_norm(act, L['down_q'], L['down_s'], down, x, self.layers[i + 1]['in_w'], h, rows, ws)
            return True
        self._linear(act, L['down_q'], L['down_s'], down, rows, ws)
        return False

    def _kernel_attention(self, qrot, kc, vc, rows, positions, pos_stride, attn):
        """Split-K attention of `rows` query rows over the shared cache (each row a batch row, batch stride 0)."""
        lib, c, st = _lib.lib(), self.cfg, self._stream()
        d = c.head_dim
        if rows == 1:
            nsplit, ws = self.nsplit, self.attn_ws
        else:
            nsplit = lib.egpt_decode_attn_default_splits(rows, c.kv_heads, self.cap)
            need = ctypes.c_size_t()
            _lib.check('egpt_decode_attn_workspace', lib.egpt_decode_attn_workspace(
                rows, c.heads, c.kv_heads, self.cap, d, nsplit, need))
            ws = torch.empty(need.value, device=self.device, dtype=torch.uint8)
        _lib.check('egpt_decode_attn', lib.egpt_decode_attn(
            _lib.EGPT_BF16, qrot.data_ptr(), qrot.stride(0), d,
            kc.data_ptr(), 0, kc.stride(0), kc.stride(1),
            vc.data_ptr(), 0, vc.stride(0), vc.stride(1),
            positions.data_ptr(), pos_stride,
            attn.data_ptr(), attn.stride(0), d,
            ws.data_ptr(), ws.numel(), rows, c.heads, c.kv_heads, self.cap, d, nsplit, d ** -0.5, st))

    def _head(self, x, down, h):
        """Final residual add + norm of one row, lm_head GEMV, argmax into token, position += 1."""
        lib, c, st = _lib.lib(), self.cfg, self._stream()
        _lib.check('egpt_add_rmsnorm', lib.egpt_add_rmsnorm(
            x.data_ptr(), x.stride(0), down.data_ptr(), down.stride(0), self.norm_w.data_ptr(), h.data_ptr(),
            h.stride(0), 1, c.hidden, c.rms_eps, st))
        self._linear(h, self.head_q, self.head_s, self.logits, 1)
        _lib.check('egpt_argmax', lib.egpt_argmax(self.logits.data_ptr(), c.vocab, self.arg_ws.data_ptr(),
                                                  self.arg_ws.numel(), self.token.data_ptr(),
                                                  self.position.data_ptr(), st))

    # ------------------------------------------------------------------ public API

    @torch.inference_mode()
    def reset(self):
        """Clear the cache and the token / position state (in place: captured addresses stay valid)."""
        self.k_cache.zero_()
        self.v_cache.zero_()
        self.token.zero_()
        self.position.zero_()

    @torch.inference_mode()
    def step(self):
        """One decode step on the current stream (egpt_qwen3_decode_step): consumes self.token at self.position,
        writes the next token; five launches per layer and one for the head."""
        _lib.check('egpt_qwen3_decode_step', _lib.lib().egpt_qwen3_decode_step(ctypes.byref(self._step_c),
                                                                               self._stream()))

    @torch.inference_mode()
    def step_unfused(self):
        """The same step with one kernel per op (embedding, norms, GEMVs, rope, attention, SwiGLU, argmax)."""
        lib, c = _lib.lib(), self.cfg
        _lib.check('egpt_embed', lib.egpt_embed(self.token.data_ptr(), 1, self.embed.data_ptr(), self.embed.stride(0),
                                                c.vocab, self.x.data_ptr(), self.x.stride(0), c.hidden,
                                                self._stream()))
        for i in range(c.layers):
            self._layer(i, 1, self.x, self.h, self.qkv, self.qrot, self.attn, self.o, self.gu, self.act, self.down,
                        self.position, 0, first=(i == 0))
        self._head(self.x, self.down, self.h)

    @torch.inference_mode()
    def prefill(self, tokens, pos0=0):
        """Run prompt ids (1-D, on any device) at positions pos0.. through the model; sets token = greedy next
        token and position = pos0 + len(tokens). Returns the last row's logits (bf16 [vocab])."""
        c, dev, bf = self.cfg, self.device, torch.bfloat16
        ids = torch.as_tensor(tokens, dtype=torch.long).reshape(-1).to(dev)
        t = ids.numel()
        if t < 1:
            raise ValueError('prefill needs at least one token')
        if pos0 + t > self.cap:
            raise ValueError('prompt exceeds the cache capacity')
        positions = torch.arange(pos0, pos0 + t, device=dev, dtype=torch.long)
        x = torch.empty(t, c.hidden, device=dev, dtype=bf)
        h = torch.empty_like(x)
        qkv = torch.empty(t, self.n_qkv, device=dev, dtype=bf)
        qrot = torch.empty(t, c.heads * c.head_dim, device=dev, dtype=bf)
        attn = torch.empty_like(qrot)
        o = torch.empty_like(x)
        gu = torch.empty(t, 2 * c.inter, device=dev, dtype=bf)
        act = torch.empty(t, c.inter, device=dev, dtype=bf)
        down = torch.empty_like(x)
        lib = _lib.lib()
        _lib.check('egpt_embed', lib.egpt_embed(ids.data_ptr(), t, self.embed.data_ptr(), self.embed.stride(0),
                                                c.vocab, x.data_ptr(), x.stride(0), c.hidden, self._stream()))
        ws = self._prefill_workspace(t) if t > MAX_DECODE_ROWS else None
        normed = False
        for i in range(c.layers):
            normed = self._layer(i, t, x, h, qkv, qrot, attn, o, gu, act, down, positions, 1, first=(i == 0),
                                 pos0=pos0, normed=normed, ws=ws)
        self.position.fill_(pos0 + t - 1)  # argmax advances it to pos0 + t
        self._head(x[t - 1:], down[t - 1:], h[t - 1:])
        return self.logits[0]

    @torch.inference_mode()
    def capture(self):
        """Capture step() as one graph (warm-up on a side stream first, as graph capture requires).

        Runs under inference mode like every other engine entry point, so the capture
        never mixes inference and normal tensors (torch's graph capture updates its
        RNG state tensors in place).
        """
        saved = (self.token.clone(), self.position.clone(), self.x.clone())
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self.step()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        torch.cuda.synchronize(self.device)
        self.token.copy_(saved[0])
        self.position.copy_(saved[1])
        self.x.copy_(saved[2])
        self.graph = g
        return g

    @torch.inference_mode()
    def replay(self):
        if self.graph is None:
            self.capture()
        self.graph.replay()
