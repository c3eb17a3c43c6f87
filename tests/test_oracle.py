"""Pins the CPU oracle (oracle/) before the HIP kernels are tested against it."""

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import int8 as oint8
from oracle.numerics import bf16_bits, from_bf16_bits, to_bf16


# ---------------------------------------------------------------- bf16 rounding

def test_bf16_known_bits_and_ties_to_even():
    # 1 + 2^-8 is exactly half-way between bf16 1.0 and 1.0078125: ties to even -> 1.0
    # 1 + 3 * 2^-8 is half-way between 1.0078125 (odd) and 1.015625 (even) -> 1.015625
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.4e38, np.inf, -0.0], np.float32)
    got = to_bf16(vals)
    assert got[0] == 1.0 and got[1] == 1.0 and got[2] == 1.015625 and got[3] == -2.5
    assert np.isinf(got[4]) and np.isinf(got[5]) and np.signbit(got[6])
    assert np.isnan(to_bf16(np.array([np.nan], np.float32)))[0]
    assert bf16_bits(np.array([1.0], np.float32))[0] == 0x3F80
    assert from_bf16_bits(np.array([0xC020], np.uint16))[0] == -2.5


def test_bf16_matches_torch_cast():
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 1e3
    ours = to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, theirs)


# ---------------------------------------------------------------- int8 quantisation

def test_quantize_known_answer_half_even():
    # max |w| = 1 -> s = 1/127; -0.5 / s = -63.5 rounds to the even -64; 0.25 / s = 31.75 -> 32
    q, s = oint8.quantize_weight(np.array([[1.0, -0.5, 0.25], [0.0, 0.0, 0.0]], np.float32))
    assert s[0] == np.float32(1.0) / np.float32(127.0)
    assert q[0].tolist() == [127, -64, 32]
    assert s[1] == np.float32(1e-12) and q[1].tolist() == [0, 0, 0]


def test_quantize_invariants_and_torch_agreement():
    # research/realmodel/test_int8_linear.py:43-53: closed form, |q|max = 127, half-step reconstruction
    rng = np.random.default_rng(1)
    w = rng.standard_normal((300, 128)).astype(np.float32)
    q, s = oint8.quantize_weight(w)
    assert q.dtype == np.int8 and int(np.abs(q.astype(np.int32)).max(axis=1).min()) == 127
    assert float(np.abs(q.astype(np.float32) * s[:, None] - w).max()) <= float(s.max()) / 2 + 1e-6
    from efficientgpt_amd.int8_linear import quantize_weight as product_quantize
    tq, ts = product_quantize(torch.from_numpy(w))
    assert np.array_equal(tq.numpy(), q) and np.array_equal(ts.numpy(), s)


def test_quantize_row_blocks_match_whole_matrix():
    from efficientgpt_amd.int8_linear import quantize_weight as product_quantize
    big = torch.randn(20000, 64, generator=torch.Generator().manual_seed(2))  # > one 8192-row block
    qb, sb = product_quantize(big)
    s_ref = (big.abs().amax(1) / 127.0).clamp_min(1e-12)
    assert torch.equal(sb, s_ref)
    assert torch.equal(qb, torch.round(big / s_ref[:, None]).clamp(-127, 127).to(torch.int8))


# ---------------------------------------------------------------- int8 linear formulas

def _int8_case(m, k, n, seed=0):
    rng = np.random.default_rng(seed)
    x = to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = (rng.random(n).astype(np.float32) * 0.02 + 1e-3).astype(np.float32)
    return x, q, s


def test_linear_decode_equals_brute_force_loops():
    x, q, s = _int8_case(3, 100, 70)
    want = np.zeros((3, 70), np.float64)
    for i in range(3):
        for j in range(70):
            acc = 0.0
            for kk in range(100):
                acc += float(x[i, kk]) * float(q[j, kk])
            want[i, j] = acc
    got = oint8.linear_decode(x, q, s)
    ref = to_bf16((want.astype(np.float32) * s[None, :]).astype(np.float32))
    assert np.array_equal(got, ref)


def test_linear_formulas_within_reference_tolerance():
    for m, k, n in [(1, 2048, 256), (4, 512, 64), (16, 256, 48), (17, 256, 32)]:
        x, q, s = _int8_case(m, k, n, seed=m)
        tol = oint8.tolerance_vs_naive(x, q, s)
        assert oint8.max_err(oint8.linear_decode(x, q, s), x, q, s) <= tol
        assert oint8.max_err(oint8.linear_prefill(x, q, s), x, q, s) <= tol
        assert oint8.max_err(oint8.linear(x, q, s), x, q, s) <= oint8.tolerance_vs_eager(x, q, s)


def test_tolerance_rejects_planted_mistakes():
    # the mutations research/kernelagent/test_evaluate.py:86-95 must reject
    x, q, s = _int8_case(1, 2048, 512, seed=3)
    tol = oint8.tolerance_vs_eager(x, q, s)
    no_scale = to_bf16((x.astype(np.float64) @ q.astype(np.float64).T).astype(np.float32))
    assert oint8.max_err(no_scale, x, q, s) > tol
    skip_last = oint8.linear_decode(x[:, :-128], q[:, :-128], s)
    assert oint8.max_err(skip_last, x, q, s) > tol
    unsigned = oint8.linear_decode(x, q.view(np.uint8).astype(np.float32), s)
    assert oint8.max_err(unsigned, x, q, s) > tol


def test_linear_row_rule():
    x, q, s = _int8_case(17, 64, 32, seed=4)
    assert np.array_equal(oint8.linear(x, q, s), oint8.linear_prefill(x, q, s))
    assert np.array_equal(oint8.linear(x[:16], q, s), oint8.linear_decode(x[:16], q, s))


# ---------------------------------------------------------------- attention

def _attn_case(b, hq, hkv, cap, d, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, hq, 1, d)) * scale
    k = rng.standard_normal((b, hkv, cap, d)) * scale
    v = rng.standard_normal((b, hkv, cap, d))
    return q, k, v


def test_attention_position_zero_returns_first_value():
    q, k, v = _attn_case(2, 4, 2, 9, 64)
    out = oatt.attention_truth(q, k, v, np.array([0, 0]))
    assert np.allclose(out[:, :, 0], np.repeat(v[:, :, 0], 2, axis=1), rtol=0, atol=1e-15)


def test_attention_constant_keys_give_mean_of_values():
    q, k, v = _attn_case(1, 4, 4, 20, 64)
    k[:] = 0.3
    out = oatt.attention_truth(q, k, v, np.array([12]))
    assert np.allclose(out[0, :, 0], v[0, :, :13].mean(axis=1), atol=1e-12)


def test_attention_gqa_equals_repeated_mha_and_torch_sdpa():
    q, k, v = _attn_case(3, 8, 2, 37, 64, seed=5, scale=2.0)
    pos = np.array([3, 36, 20])
    gqa = oatt.attention_truth(q, k, v, pos)
    mha = oatt.attention_truth(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), pos)
    assert np.array_equal(gqa, mha)
    tq, tk, tv = (torch.from_numpy(a) for a in (q, np.repeat(k, 4, 1), np.repeat(v, 4, 1)))
    allowed = torch.arange(37).view(1, 1, 1, 37) <= torch.from_numpy(pos).view(-1, 1, 1, 1)
    sdpa = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=allowed).numpy()
    assert np.allclose(gqa, sdpa, atol=1e-12, rtol=0)


def test_attention_splitk_restatement_tracks_truth_and_ignores_poison():
    q, k, v = _attn_case(2, 4, 2, 80, 64, seed=6, scale=8.0)
    pos = np.array([0, 61])
    truth = oatt.attention_truth(q, k, v, pos)
    for split, block in ((16, 16), (64, 32), (80, 80)):
        got = oatt.attention_splitk(q, k, v, pos, split=split, block_n=block)
        assert np.abs(got - truth).max() < 1e-5
    poisoned_k, poisoned_v = k.copy(), v.copy()
    for b, p in enumerate(pos):
        poisoned_k[b, :, p + 1:] = np.nan
        poisoned_v[b, :, p + 1:] = np.nan
    assert np.array_equal(oatt.attention_splitk(q, poisoned_k, poisoned_v, pos), oatt.attention_splitk(q, k, v, pos))


def test_attention_mask_off_by_one_is_caught():
    # reading one slot past the position (research/kernelagent/test_evaluate.py:45-48) must exceed the tolerance
    q, k, v = _attn_case(1, 4, 2, 64, 64, seed=7)
    pos = np.array([30])
    truth = oatt.attention_truth(q, k, v, pos)
    wrong = oatt.attention_truth(q, k, v, pos + 1)
    assert np.abs(wrong - truth).max() > 1e-3


def test_prefill_truth_rows_equal_decode_attention_and_causal_sdpa():
    # row t of a prompt block at pos0 is the decode attention at position pos0 + t over the same cache
    rng = np.random.default_rng(8)
    hq, hkv, cap, d, pos0, rows = 8, 2, 50, 32, 13, 29
    q = rng.standard_normal((rows, hq, d)) * 2.0
    k = rng.standard_normal((hkv, cap, d)) * 2.0
    v = rng.standard_normal((hkv, cap, d))
    got = oatt.prefill_truth(q, k, v, pos0)
    per_row = oatt.attention_truth(q[:, :, None, :], np.repeat(k[None], rows, 0), np.repeat(v[None], rows, 0),
                                   pos0 + np.arange(rows))
    assert np.allclose(got, per_row[:, :, 0], atol=1e-12, rtol=0)
    # from position 0 over exactly `rows` slots it is torch's causal SDPA (is_causal), repeat_kv applied
    got0 = oatt.prefill_truth(q, k, v, 0)
    tq = torch.from_numpy(q).permute(1, 0, 2)
    tk = torch.from_numpy(np.repeat(k[:, :rows], hq // hkv, 0))
    tv = torch.from_numpy(np.repeat(v[:, :rows], hq // hkv, 0))
    sdpa = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True).permute(1, 0, 2).numpy()
    assert np.allclose(got0, sdpa, atol=1e-12, rtol=0)
    # the mask shifted by one slot (each row also seeing the next slot) is caught
    assert np.abs(oatt.prefill_truth(q, k, v, pos0 + 1) - got).max() > 1e-3


# ---------------------------------------------------------------- Qwen3 step vs transformers

def _fp32_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """transformers attention hook with the decode kernel's contract: fp32 math, causal over the cache."""
    g = query.shape[1] // key.shape[1]
    k = key.float().repeat_interleave(g, 1)
    v = value.float().repeat_interleave(g, 1)
    s = (query.float() @ k.transpose(-1, -2)) * scaling
    t, n = s.shape[-2], s.shape[-1]
    allowed = torch.arange(n)[None, :] <= (n - t + torch.arange(t))[:, None]
    s = s.masked_fill(~allowed, float('-inf'))
    return (torch.softmax(s, -1) @ v).to(query.dtype).transpose(1, 2).contiguous(), None


@pytest.fixture(scope='module')
def tiny_hf():
    transformers = pytest.importorskip('transformers')
    transformers.AttentionInterface.register('egpt_fp32_test', _fp32_attention)
    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                                   max_position_embeddings=256, tie_word_embeddings=True, initializer_range=0.2,
                                   attn_implementation='egpt_fp32_test')
    return transformers, cfg


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_qwen3_oracle_matches_transformers(tiny_hf, dtype):
    from oracle.qwen3 import TINY, Qwen3Oracle
    transformers, cfg = tiny_hf
    torch.manual_seed(0)
    model = transformers.Qwen3ForCausalLM(cfg).to(dtype).eval()
    with torch.no_grad():  # jitter the norm weights so a swapped q/k norm shows
        for name, p in model.named_parameters():
            if 'norm' in name:
                p.add_((0.1 * torch.randn(p.shape)).to(dtype))
    orc = Qwen3Oracle(TINY, model.state_dict(), dtype=dtype, cap=128, inv_freq=model.model.rotary_emb.inv_freq)
    g = torch.Generator().manual_seed(1)
    for p in (1, 5, 37):
        x = torch.randint(0, 512, (1, p), generator=g)
        with torch.no_grad():
            want = model.generate(input_ids=x, attention_mask=torch.ones_like(x), max_new_tokens=24,
                                  min_new_tokens=24, do_sample=False, pad_token_id=0)[0, p:].tolist()
            hf_logits = model(x, logits_to_keep=1).logits[0, -1].float()
        got = orc.greedy(x[0], 24)
        assert len(set(got)) > 8
        assert got == want, (dtype, p)
        orc.reset()
        diff = float((orc.forward(x[0], 0).float() - hf_logits).abs().max())
        assert diff <= (0.0 if dtype == torch.bfloat16 else 1e-4), diff


def test_qwen3_oracle_int8_rule_uses_decode_and_prefill_formulas():
    from oracle.qwen3 import Linear
    g = torch.Generator().manual_seed(3)
    q = torch.randint(-127, 128, (48, 64), generator=g, dtype=torch.int8)
    s = torch.rand(48, generator=g) * 0.01 + 1e-3
    lin = Linear(qweight=q, scale=s)
    for rows in (1, 16, 17, 40):
        x = torch.randn(rows, 64, generator=g).to(torch.bfloat16)
        got = lin(x).float().numpy()
        want = oint8.linear(x.float().numpy(), q.numpy(), s.numpy())
        assert np.array_equal(got, want), rows
        # the forced decode rule: every row by the single-row formula, whatever the row count
        forced = lin(x, 'decode').float().numpy()
        assert np.array_equal(forced, oint8.linear_decode(x.float().numpy(), q.numpy(), s.numpy())), rows


# ---------------------------------------------------------------- RoPE frequencies and tables vs transformers

ROPE_CASES = [  # (rope_theta, head_dim, hidden, heads, kv_heads, slots)
    (1e6, 128, 2048, 16, 8, 4096),   # Qwen3-1.7B
    (1e6, 128, 4096, 32, 8, 8704),   # Qwen3-8B at the long-context cache
    (1e4, 32, 128, 4, 2, 256),       # the reference's tiny test model (transformers' default theta)
]


@pytest.mark.parametrize('theta,d,hidden,heads,kv,slots', ROPE_CASES)
def test_rope_frequencies_and_tables_match_transformers(theta, d, hidden, heads, kv, slots):
    """default_inv_freq and both rope_tables (the oracle's and the engine's, built on the host) against
    transformers' Qwen3RotaryEmbedding (compute_default_rope_parameters, then its fp32 forward cast to bf16),
    bit for bit; a planted wrong theta or a frequency index off by one must differ."""
    transformers = pytest.importorskip('transformers')
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    from efficientgpt_amd.qwen3 import Qwen3Config
    from efficientgpt_amd.qwen3 import rope_tables as engine_rope_tables
    from oracle.qwen3 import Qwen3Shape, default_inv_freq, rope_tables

    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=hidden, intermediate_size=256, num_hidden_layers=1,
                                   num_attention_heads=heads, num_key_value_heads=kv, head_dim=d, rope_theta=theta,
                                   max_position_embeddings=slots)
    rot = Qwen3RotaryEmbedding(cfg)
    shape = Qwen3Shape(vocab=512, hidden=hidden, inter=256, layers=1, heads=heads, kv_heads=kv, head_dim=d,
                       rope_theta=theta)
    inv = default_inv_freq(shape)
    assert inv.dtype == rot.inv_freq.dtype == torch.float32
    assert torch.equal(inv, rot.inv_freq)
    x = torch.zeros(1, 1, d, dtype=torch.bfloat16)
    want_cos, want_sin = rot(x, torch.arange(slots)[None])
    cos, sin = rope_tables(shape, slots, torch.bfloat16)
    assert torch.equal(cos, want_cos[0]) and torch.equal(sin, want_sin[0])
    ecfg = Qwen3Config.from_hf(cfg)
    assert ecfg.rope_theta == theta and ecfg.head_dim == d
    ecos, esin = engine_rope_tables(ecfg, slots)
    assert torch.equal(ecos, want_cos[0]) and torch.equal(esin, want_sin[0])
    # planted mistakes: theta off by a factor 10, the exponent's index shifted by one
    wrong_theta = Qwen3Shape(vocab=512, hidden=hidden, inter=256, layers=1, heads=heads, kv_heads=kv, head_dim=d,
                             rope_theta=theta * 10)
    assert not torch.equal(default_inv_freq(wrong_theta), rot.inv_freq)
    shifted = 1.0 / (theta ** (torch.arange(1, d + 1, 2, dtype=torch.float) / d))
    assert not torch.equal(shifted, rot.inv_freq)
    assert not torch.equal(rope_tables(wrong_theta, slots, torch.bfloat16)[0], want_cos[0])


# ---------------------------------------------------------------- teacher-forced batch form of the oracle

@pytest.mark.parametrize('shape_name', ['TINY', 'SMALL'])
def test_oracle_teacher_forced_rows_equal_sequential_decode(shape_name):
    """forward(tokens, pos, all_logits=True, rule='decode') computes in one pass what len(tokens) single-token
    decode steps compute. The rows differ from the sequential steps only by fp32 summation order inside the
    matrix products (one bf16 ulp in an activation, carried through the layers): within 1e-2 of the largest
    logit, the same greedy pick (a near-tie aside) and the same cache. Planted mistakes move further off: the
    prefill rule on the 24 rows (double rounding), and positions shifted by one (RoPE and the causal mask).
    The chunked attention of a long prompt equals the unchunked form within the same bound."""
    from oracle.qwen3 import TINY, Qwen3Oracle, Qwen3Shape, quantize_weights, random_weights
    from tests.near_tie import near_tie_bound
    shape = TINY if shape_name == 'TINY' else Qwen3Shape(vocab=1024, hidden=512, inter=1024, layers=2, heads=16,
                                                          kv_heads=8, head_dim=128)
    w = quantize_weights(random_weights(shape, seed=5, std=0.15, norm_jitter=0.1), shape)
    g = torch.Generator().manual_seed(6)
    prompt = torch.randint(0, shape.vocab, (40,), generator=g)
    forced = torch.randint(0, shape.vocab, (24,), generator=g)

    def primed():
        o = Qwen3Oracle(shape, w, cap=96)
        o.forward(prompt, 0)
        return o

    seq = primed()
    want = torch.stack([seq.forward([int(t)], 40 + i) for i, t in enumerate(forced)]).float()
    scale = float(want.abs().max())
    bat = primed()
    got = bat.forward(forced, 40, all_logits=True, rule='decode').float()
    rel = float((got - want).abs().max()) / scale
    assert float((got[0] - want[0]).abs().max()) == 0.0  # the first row sees the same cache in both forms
    assert rel <= 1e-2, rel
    for i in range(len(forced)):
        a, b = int(torch.argmax(got[i])), int(torch.argmax(want[i]))
        assert a == b or float(want[i, b] - want[i, a]) < near_tie_bound(float(want[i, b])), i
    for L in range(shape.layers):
        kb, ks = bat.k_cache[L].float(), seq.k_cache[L].float()
        assert float((kb - ks).abs().max()) <= 1e-2 * float(ks.abs().max())
    off_rule = float((primed().forward(forced, 40, all_logits=True).float() - want).abs().max()) / scale
    off_pos = float((primed().forward(forced, 41, all_logits=True, rule='decode').float() - want).abs().max()) / scale
    assert off_rule > rel and off_pos > 0.1, (off_rule, off_pos)
    # chunked attention (chunk 7) against one chunk covering every row
    l1 = Qwen3Oracle(shape, w, cap=96).forward(prompt, 0, all_logits=True).float()
    o2 = Qwen3Oracle(shape, w, cap=96)
    o2._attention = (lambda q, layer, pos0, f=o2._attention: f(q, layer, pos0, chunk=7))
    l2 = o2.forward(prompt, 0, all_logits=True).float()
    assert float((l1 - l2).abs().max()) <= 1e-2 * float(l1.abs().max())


def test_oracle_splitk_sum_is_another_fp32_order_of_the_same_product():
    """Linear.ksplit (the reference's split-K GEMV, research/realmodel/int8_linear.py:41-64): chunks of
    KCHUNK = ceil(ceil(K / splits) / 128) * 128 columns. Pinned by: integer-valued inputs (every fp32 partial sum
    exact) give the one-pass result bit for bit, whatever the chunking; each chunk boundary matters (zeroing the
    columns past the first chunk leaves exactly the first chunk's one-pass product, which a boundary anywhere but
    at 256 would change); random inputs stay within fp32 rounding of
    the fp64 truth and round to the same bf16 as the one-pass form on all but a few outputs."""
    from oracle.qwen3 import Linear
    g = torch.Generator().manual_seed(11)
    k, n = 300, 96
    q = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = torch.rand(n, generator=g) * 0.01 + 1e-3
    one, two, three = Linear(qweight=q, scale=s), Linear(qweight=q, scale=s, ksplit=2), \
        Linear(qweight=q, scale=s, ksplit=3)
    xi = torch.randint(-8, 9, (4, k), generator=g).to(torch.bfloat16)
    assert torch.equal(one(xi, 'decode'), two(xi, 'decode')) and torch.equal(one(xi, 'decode'), three(xi, 'decode'))
    # ksplit 2 at K = 300: KCHUNK = 256, chunks [0, 256) and [256, 300)
    x = torch.randn(5, k, generator=g).to(torch.bfloat16)
    two(x, 'decode')  # builds the cached image
    head = x.clone()
    head[:, 256:] = 0
    assert torch.equal(two._sum(head), x[:, :256].float() @ q[:, :256].float().t())
    assert not torch.equal(two._sum(x), one._sum(x))  # a different order: some sums round differently
    truth = x.double() @ q.double().t()
    for lin in (two, three):
        acc = lin._sum(x).double()
        bound = k * 2.0 ** -23 * (x.double().abs() @ q.double().abs().t())
        assert bool(((acc - truth).abs() <= bound).all())
        same = (lin(x, 'decode') == one(x, 'decode')).float().mean()
        assert float(same) >= 0.97, float(same)
