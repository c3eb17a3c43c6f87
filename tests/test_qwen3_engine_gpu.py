"""Qwen3 int8 decode engine and graph decoder vs the CPU oracle.

Mirrors research/realmodel/test_fast_decode.py (tiny random Qwen3 with 4 query /
2 kv heads, prompts of 1, 5 and 37 tokens, 40 new tokens, non-degenerate output,
EOS exactness without leaking run-ahead tokens, cache reset between requests,
guards) with the CPU oracle (oracle/qwen3.py, pinned against transformers) as the
reference, and adds a Qwen3-shaped layer at the real head geometry (D = 128).
"""

import numpy as np
import pytest
import torch

from oracle.qwen3 import Qwen3Oracle, Qwen3Shape, TINY, quantize_weights, random_weights
from tests.near_tie import near_tie_bound, near_tie_match

pytestmark = pytest.mark.gpu

# Qwen3-1.7B head geometry (16 q / 8 kv heads, D = 128) at a small width and depth
SMALL = Qwen3Shape(vocab=2048, hidden=512, inter=1024, layers=3, heads=16, kv_heads=8, head_dim=128)
# Qwen3-1.7B widths (hidden 2048, intermediate 6144, vocab 151936) at two layers
WIDE2 = Qwen3Shape(vocab=151936, hidden=2048, inter=6144, layers=2, heads=16, kv_heads=8, head_dim=128)
# Qwen3-8B head geometry (32 q / 8 kv heads: 4 query heads per kv head, o_proj over 4096 inputs) at a small width
SMALL8 = Qwen3Shape(vocab=2048, hidden=512, inter=1024, layers=3, heads=32, kv_heads=8, head_dim=128)
# Qwen3-8B widths (hidden 4096, intermediate 12288, 32 / 8 heads) at two layers and a short vocabulary
WIDE8 = Qwen3Shape(vocab=4096, hidden=4096, inter=12288, layers=2, heads=32, kv_heads=8, head_dim=128)


def build(shape, seed, std, cap):
    from efficientgpt_amd.qwen3 import Qwen3Config, Qwen3Int8Engine
    w = quantize_weights(random_weights(shape, seed=seed, std=std, norm_jitter=0.1), shape)
    cfg = Qwen3Config(shape.vocab, shape.hidden, shape.inter, shape.layers, shape.heads, shape.kv_heads,
                      shape.head_dim, shape.rope_theta, shape.rms_eps, shape.tied)
    eng = Qwen3Int8Engine(cfg, {k: v.cuda() for k, v in w.items()}, cap)
    orc = Qwen3Oracle(shape, w, dtype=torch.bfloat16, cap=cap)
    return eng, orc


def oracle_greedy_with_margins(orc, prompt, n):
    toks, margins = orc.greedy(prompt, n, with_margins=True)
    orc.reset()
    tops, logits, pos = [], orc.forward(prompt, 0), len(prompt)
    for i in range(n):
        tops.append(float(logits.float().max()))
        if i + 1 < n:
            logits = orc.forward([toks[i]], pos)
            pos += 1
    return toks, margins, tops


@pytest.mark.parametrize('shape,std', [(TINY, 0.2), (SMALL, 0.15)])
def test_prefill_logits_match_oracle(shape, std):
    eng, orc = build(shape, seed=1, std=std, cap=224)
    g = torch.Generator().manual_seed(2)
    for p in (1, 5, 17, 37, 100, 200):  # 100 rows: the decode kernel over the prompt; 200: the prompt kernel
        prompt = torch.randint(0, shape.vocab, (p,), generator=g)
        eng.reset()
        got = eng.prefill(prompt).float().cpu()
        orc.reset()
        want = orc.forward(prompt, 0).float()
        rel = float((got - want).abs().max() / want.abs().max())
        assert rel < 2e-2, (p, rel)
        assert int(torch.argmax(got)) == int(torch.argmax(want)) or \
            float(want.max() - want[int(torch.argmax(got))]) < 0.1 * float(want.abs().max()), p


def teacher_forced_agreement(eng, prompt, ref, margins, tops):
    """Per-step greedy agreement with the oracle's own tokens fed back (no divergence cascade).

    Returns (agreeing steps, steps, non-near-tie disagreements)."""
    eng.reset()
    eng.prefill(prompt)
    got = [int(eng.token)]
    for i in range(1, len(ref)):
        eng.token.fill_(ref[i - 1])
        eng.replay()
        got.append(int(eng.token))
    bad = [i for i, (a, b) in enumerate(zip(ref, got)) if a != b and margins[i] >= near_tie_bound(tops[i])]
    return sum(a == b for a, b in zip(ref, got)), len(ref), bad


@pytest.mark.parametrize('shape,std', [(TINY, 0.2), (SMALL, 0.15)])
def test_graph_decoder_greedy_matches_oracle(shape, std):
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    eng, orc = build(shape, seed=3, std=std, cap=128)
    dec = GraphGreedyDecoder(eng, max_cache_len=128)
    g = torch.Generator().manual_seed(1)
    agree = total = 0
    for p in (1, 5, 37):
        x = torch.randint(0, shape.vocab, (1, p), generator=g)
        got, st = dec.generate(x.cuda(), 40)
        assert st['tokens'] == 40 and len(got) == 40
        assert len(set(got)) > 8, 'degenerate model output would make equality trivial'
        ref, margins, tops = oracle_greedy_with_margins(orc, x[0], 40)
        # free-running: equal, or first divergence at a near-tie (the reference's rule)
        ok, where = near_tie_match(ref, got, margins, tops)
        assert ok, (p, where, ref[:where + 1] if where is not None else None, got[:where + 1] if where else None)
        # teacher-forced: every step's greedy pick agrees unless that step is a near-tie
        a, n, bad = teacher_forced_agreement(eng, x[0], ref, margins, tops)
        assert not bad, (p, bad)
        agree += a
        total += n
    assert agree / total >= 0.95, agree / total


@pytest.mark.parametrize('shape,std,cap,plen', [(TINY, 0.2, 96, 9), (SMALL, 0.15, 96, 9), (SMALL, 0.15, 2048, 9),
                                                (SMALL, 0.15, 2048, 1500), (TINY, 0.2, 4096, 9),
                                                (TINY, 0.2, 8192, 9), (SMALL8, 0.15, 96, 9),
                                                (SMALL8, 0.15, 2048, 1500), (SMALL8, 0.15, 4096, 9),
                                                (SMALL8, 0.15, 4096, 3000), (SMALL, 0.15, 3072, 2900),
                                                (SMALL8, 0.15, 3072, 2900)])
def test_fused_step_matches_unfused_step(shape, std, cap, plen):
    """The fused step against the one-kernel-per-op step on the same tokens. Up to 3072 slots the attention blocks
    serve one query head and the o_proj GEMV merges their 2 or 8 splits (a 1500-token prompt fills the 8 splits of
    a 2048-slot cache: about 190 slots each; a 2900-token prompt 8 of about 360 in a 3072-slot cache); at 4096 slots (32 splits, TINY 64; 8192 slots, TINY 128) the blocks
    serve a kv head's whole group and a launch of its own merges the splits, and a 3000-token prompt fills most of
    the 32 splits. SMALL8 runs 4 query heads per kv head, as Qwen3-8B does."""
    eng, _ = build(shape, seed=11, std=std, cap=cap)
    prompt = torch.randint(0, shape.vocab, (plen,), generator=torch.Generator().manual_seed(3))
    runs = {}
    for name, fn in (('unfused', eng.step_unfused), ('fused', eng.step)):
        eng.reset()
        eng.prefill(prompt)
        toks, logits = [], []
        forced = runs.get('unfused', (None,))[0]
        for i in range(12):
            if forced is not None and i > 0:
                eng.token.fill_(forced[i - 1])  # same inputs even past a near-tie
            fn()
            toks.append(int(eng.token))
            logits.append(eng.logits[0].float().cpu().clone())
        torch.cuda.synchronize()
        runs[name] = (toks, logits, eng.k_cache.float().cpu().clone(), eng.v_cache.float().cpu().clone(),
                      int(eng.position))
    (tu, lu, ku, vu, pu), (tf, lf, kf, vf, pf) = runs['unfused'], runs['fused']
    assert pu == pf == plen + 12
    for a, b in zip(lu, lf):
        assert float((a - b).abs().max()) <= 2e-2 * float(a.abs().max())
    assert float((ku - kf).abs().max()) <= 2e-2 * float(ku.abs().max())
    assert torch.equal(vu[:, :, :plen], vf[:, :, :plen])  # prompt slots come from the same prefill
    assert float((vu - vf).abs().max()) <= 2e-2 * float(vu.abs().max())
    agree = sum(a == b for a, b in zip(tu, tf))
    assert agree >= 11, (tu, tf)


@pytest.mark.parametrize('shape', [SMALL, SMALL8])
@pytest.mark.parametrize('plen', [40, 128, 4096])
def test_prefill_folded_norms_equal_separate_calls(shape, plen):
    """Prompts of 17-128 rows take the split-K GEMM for o_proj and down_proj, with the residual add + RMSNorm folded
    into its reduce (egpt_int8_gemm_add_rmsnorm) and each down projection also taking the next layer's input norm
    (the first layer normalises its embedding rows itself; the last leaves x + down to the head); a 4096-row prompt
    takes SwiGLU in the gate/up GEMM's epilogue (egpt_int8_gemm_swiglu). The same prompt with the folds turned off
    (separate linear, egpt_add_rmsnorm and egpt_silu_mul calls, each layer normalising its own input) must give the
    same logits and the same K/V caches, bit for bit."""
    eng, _ = build(shape, seed=9, std=0.15, cap=max(160, plen + 8))
    prompt = torch.randint(0, shape.vocab, (plen,), generator=torch.Generator().manual_seed(plen))
    out = []
    for fold in (True, False):
        eng.fold_norms = fold
        eng.reset()
        logits = eng.prefill(prompt).clone()
        out.append((logits, eng.k_cache.clone(), eng.v_cache.clone(), int(eng.token), int(eng.position)))
    (la, ka, va, ta, pa), (lb, kb, vb, tb, pb) = out
    assert torch.equal(la, lb)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert (ta, pa) == (tb, pb) and pa == plen


def test_qwen3_1p7b_widths_match_oracle():
    """Real Qwen3-1.7B widths (hidden 2048, inter 6144, vocab 151936, 16/8 heads) at two layers:
    prefill logits and teacher-forced greedy steps of the fused step against the CPU oracle."""
    eng, orc = build(WIDE2, seed=21, std=0.05, cap=64)
    prompt = torch.randint(0, WIDE2.vocab, (16,), generator=torch.Generator().manual_seed(5))
    ref, margins, tops = oracle_greedy_with_margins(orc, prompt, 12)
    assert len(set(ref)) > 4
    a, n, bad = teacher_forced_agreement(eng, prompt, ref, margins, tops)
    assert not bad, bad
    assert a >= n - 1, (a, n)
    # logits of the last teacher-forced step against the oracle's
    orc.reset()
    logits, pos = orc.forward(prompt, 0), len(prompt)
    for t in ref[:-1]:
        logits = orc.forward([t], pos)
        pos += 1
    got = eng.logits[0].float().cpu()
    want = logits.float()
    assert float((got - want).abs().max()) <= 2e-2 * float(want.abs().max())


def test_qwen3_8b_widths_match_oracle():
    """Qwen3-8B widths (hidden 4096, inter 12288, 32 / 8 heads) at two layers: teacher-forced greedy steps of the
    fused step against the CPU oracle, and the last step's logits, with attention blocks of one query head (64 slots,
    splits merged in the o_proj GEMV) and of a kv head's whole group (4096 slots, 32 splits: the separate merge
    launch)."""
    for cap in (64, 4096):
        eng, orc = build(WIDE8, seed=23, std=0.03, cap=cap)
        prompt = torch.randint(0, WIDE8.vocab, (11,), generator=torch.Generator().manual_seed(6))
        ref, margins, tops = oracle_greedy_with_margins(orc, prompt, 8)
        assert len(set(ref)) > 3
        a, n, bad = teacher_forced_agreement(eng, prompt, ref, margins, tops)
        assert not bad, (cap, bad)
        assert a >= n - 1, (cap, a, n)
        orc.reset()
        logits, pos = orc.forward(prompt, 0), len(prompt)
        for t in ref[:-1]:
            logits = orc.forward([t], pos)
            pos += 1
        got = eng.logits[0].float().cpu()
        want = logits.float()
        assert float((got - want).abs().max()) <= 2e-2 * float(want.abs().max()), cap
        del eng, orc
        torch.cuda.empty_cache()


@pytest.mark.parametrize('shape', [SMALL, SMALL8])
def test_long_prompt_in_2048_slots_matches_oracle(shape):
    """A 1500-token prompt in a 2048-slot cache: the step's 8 splits of one-query-head blocks each hold about 190
    slots, merged in the o_proj GEMV. Teacher-forced greedy steps and the last step's logits against the oracle."""
    eng, orc = build(shape, seed=29, std=0.15, cap=2048)
    prompt = torch.randint(0, shape.vocab, (1500,), generator=torch.Generator().manual_seed(8))
    ref, margins, tops = oracle_greedy_with_margins(orc, prompt, 10)
    assert len(set(ref)) > 4
    a, n, bad = teacher_forced_agreement(eng, prompt, ref, margins, tops)
    assert not bad, bad
    assert a >= n - 1, (a, n)
    orc.reset()
    logits, pos = orc.forward(prompt, 0), len(prompt)
    for t in ref[:-1]:
        logits = orc.forward([t], pos)
        pos += 1
    got = eng.logits[0].float().cpu()
    want = logits.float()
    assert float((got - want).abs().max()) <= 2e-2 * float(want.abs().max())


@pytest.mark.parametrize('shape,cap', [(SMALL, 96), (SMALL8, 96), (SMALL, 2048), (SMALL8, 4096), (TINY, 8192)])
def test_fused_step_ignores_cache_past_position(shape, cap):
    """NaN in every cache slot past the position leaves the fused step's logits bit-identical: the reference's
    poisoning test of its split kernel (research/phase5/test_graph_gpu.py:250-261) run on the whole step, through
    the o_proj merge (2 and 8 splits) with attention blocks of one query head, and the separate merge launch (32
    and 128 splits) with blocks of a kv head's whole group."""
    eng, _ = build(shape, seed=13, std=0.15, cap=cap)
    prompt = torch.randint(0, shape.vocab, (9,), generator=torch.Generator().manual_seed(4))
    runs = []
    for fill in (0.0, float('nan')):
        eng.reset()
        eng.prefill(prompt)
        eng.k_cache[:, :, len(prompt):] = fill
        eng.v_cache[:, :, len(prompt):] = fill
        logits = []
        for _ in range(6):
            eng.step()
            logits.append(eng.logits[0].clone())
        torch.cuda.synchronize()
        runs.append(logits)
    assert all(torch.equal(a, b) for a, b in zip(*runs))
    assert not any(bool(torch.isnan(a.float()).any()) for a in runs[0])


def test_graph_replay_equals_eager_step():
    eng, _ = build(SMALL, seed=5, std=0.05, cap=64)
    prompt = torch.arange(7) * 13
    eng.reset()
    eng.prefill(prompt)
    eager = []
    for _ in range(10):
        eng.step()
        eager.append(int(eng.token))
    eng.capture()
    eng.reset()
    eng.prefill(prompt)
    graphed = []
    for _ in range(10):
        eng.replay()
        graphed.append(int(eng.token))
    assert graphed == eager


def test_eos_stops_exactly_and_never_leaks_lookahead_tokens():
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    eng, _ = build(TINY, seed=7, std=0.2, cap=128)
    dec = GraphGreedyDecoder(eng, max_cache_len=128, lookahead=8)
    x = torch.randint(0, 512, (1, 7), generator=torch.Generator().manual_seed(2)).cuda()
    full, _ = dec.generate(x, 60)
    k = max(i for i in range(len(full)) if full[i] not in full[:i])
    assert k > 10, 'EOS must fall well past the first lookahead window'
    streamed = []
    got, st = dec.generate(x, 60, eos_ids={full[k]}, on_token=streamed.append)
    assert got == full[:k + 1]
    assert streamed == got
    again, _ = dec.generate(x, 60)
    assert again == full


def test_decoder_pool_buckets_share_weights_and_match_a_single_decoder():
    """DecoderPool (the reference's capacity buckets, assistant/backends.py:232-249): each request runs on the
    smallest bucket that holds it, every bucket's engine shares the weight tensors, the least recently used decoder
    is dropped past max_decoders, and the tokens equal a plain graph decoder's at the same capacity."""
    from efficientgpt_amd.fast_decode import DecoderPool, GraphGreedyDecoder
    eng, _ = build(TINY, seed=9, std=0.2, cap=128)
    pool = DecoderPool(eng, limit=512, buckets=(64, 128, 256), max_decoders=2)
    g = torch.Generator().manual_seed(11)
    requests = [(5, 20, 64), (37, 60, 128), (5, 200, 256), (9, 30, 64), (37, 60, 128)]
    for p, n, cap in requests:
        x = torch.randint(0, TINY.vocab, (1, p), generator=g).cuda()
        got, st = pool.generate(x, n)
        assert st['capacity'] == cap and st['tokens'] == n and len(got) == n
        dec = pool.decoders[cap]
        assert dec.engine.layers is eng.layers and dec.engine.head_q is eng.head_q
        assert dec.engine.cap == cap
        assert len(pool.decoders) <= 2
        want, _ = GraphGreedyDecoder(eng.with_capacity(cap), cap).generate(x, n)  # an engine of its own
        assert got == want, (p, n, cap)
    assert list(pool.decoders) == [64, 128]  # 256 was the least recently used when 128 came back
    with pytest.raises(ValueError):
        pool.generate(torch.zeros((1, 400), dtype=torch.long, device='cuda'), 200)


def test_generate_streams_tokens_from_the_step_ring():
    """Each graph replay stores its token to the engine's pinned token ring (slot new position % capacity), which
    generate() reads instead of launching a copy per token; with the ring switched off the decoder copies every
    token, and the two runs hand out the same tokens."""
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    eng, _ = build(SMALL, seed=6, std=0.15, cap=96)
    assert eng._ring_dev, 'pinned memory not mapped for the device'
    prompt = torch.randint(0, SMALL.vocab, (1, 11), generator=torch.Generator().manual_seed(12))
    dec = GraphGreedyDecoder(eng, max_cache_len=96, lookahead=3)
    got, st = dec.generate(prompt.cuda(), 40)
    assert st['tokens'] == 40
    plen = prompt.shape[1]
    assert [int(eng.token_ring[(plen + k) % eng.cap]) for k in range(1, 40)] == got[1:]
    ring_dev = eng._ring_dev
    eng._ring_dev = None  # the decoder's copy-per-token path
    try:
        again, _ = dec.generate(prompt.cuda(), 40)
    finally:
        eng._ring_dev = ring_dev
    assert again == got


def test_guards():
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    eng, _ = build(TINY, seed=0, std=0.2, cap=32)
    dec = GraphGreedyDecoder(eng, max_cache_len=32)
    with pytest.raises(ValueError):
        dec.generate(torch.zeros((1, 20), dtype=torch.long, device='cuda'), 20)
    with pytest.raises(ValueError):
        dec.generate(torch.zeros((2, 4), dtype=torch.long, device='cuda'), 4)
    with pytest.raises(ValueError):
        dec.generate(torch.zeros((1, 4), dtype=torch.long, device='cuda'), 0)
    out, st = dec.generate(torch.zeros((1, 4), dtype=torch.long, device='cuda'), 3)
    assert (len(out), st['tokens']) == (3, 3)
    assert 'capture_s' in st


def test_transformers_model_int8_through_graph_decoder():
    """A transformers Qwen3 quantised with quantize_model decodes through the engine like the oracle."""
    transformers = pytest.importorskip('transformers')
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    from efficientgpt_amd.int8_linear import quantize_model
    torch.manual_seed(0)
    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                                   max_position_embeddings=256, tie_word_embeddings=True, initializer_range=0.2)
    model = transformers.Qwen3ForCausalLM(cfg).cuda().to(torch.bfloat16).eval()
    quantize_model(model)
    sd = {k: v.cpu() for k, v in model.state_dict().items()}
    orc = Qwen3Oracle(TINY, sd, dtype=torch.bfloat16, cap=128, inv_freq=model.model.rotary_emb.inv_freq)
    dec = GraphGreedyDecoder(model, max_cache_len=128)
    g = torch.Generator().manual_seed(1)
    for p in (1, 5, 37):
        x = torch.randint(0, 512, (1, p), generator=g)
        got, _ = dec.generate(x.cuda(), 40)
        assert len(set(got)) > 8
        ref, margins, tops = oracle_greedy_with_margins(orc, x[0], 40)
        ok, where = near_tie_match(ref, got, margins, tops)
        assert ok, (p, where)
    # a decoder of another capacity over the same model (the reference's HFBackend builds one per bucket) shares
    # the weight tensors and decodes the same tokens at the same capacity's arithmetic
    dec256 = GraphGreedyDecoder(model, max_cache_len=256)
    assert dec256.engine.layers is dec.engine.layers and dec256.engine.cap == 256
    assert GraphGreedyDecoder(model, max_cache_len=128).engine is dec.engine
    again, _ = dec256.generate(x.cuda(), 40)
    ok, where = near_tie_match(ref, again, margins, tops)
    assert ok, where


def test_hf_attention_adapter_matches_oracle_attention():
    """transformers with attn_implementation 'egpt_decode' (the HIP kernel) vs the fp32 oracle attention. The
    100-token prompt runs the split-K decode kernel over its rows; the 170-token one is past the decode kernel's
    context bound (qwen3.use_prompt_kernel): its prefill runs the prompt-attention kernel at head dim 32."""
    transformers = pytest.importorskip('transformers')
    from efficientgpt_amd import hf
    hf.register()
    torch.manual_seed(0)
    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                                   max_position_embeddings=256, tie_word_embeddings=True, initializer_range=0.2,
                                   attn_implementation=hf.NAME)
    model = transformers.Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    orc = Qwen3Oracle(TINY, sd, dtype=torch.bfloat16, cap=256, inv_freq=model.model.rotary_emb.inv_freq)
    model = model.cuda()
    g = torch.Generator().manual_seed(4)
    for p in (1, 6, 30, 100, 170):
        x = torch.randint(0, 512, (1, p), generator=g)
        with torch.no_grad():
            got = model.generate(input_ids=x.cuda(), attention_mask=torch.ones_like(x).cuda(), max_new_tokens=20,
                                 min_new_tokens=20, do_sample=False, pad_token_id=0)[0, p:].tolist()
        ref, margins, tops = oracle_greedy_with_margins(orc, x[0], 20)
        ok, where = near_tie_match(ref, got, margins, tops)
        assert ok, (p, where)


def test_engine_from_int8_checkpoint_decodes_identically(tmp_path):
    """save_engine -> Qwen3Int8Engine.from_int8: the same stored bytes, so the same logits and tokens, bit for bit."""
    import os
    from efficientgpt_amd import checkpoint
    from efficientgpt_amd.qwen3 import Qwen3Int8Engine
    eng, _ = build(SMALL, seed=4, std=0.15, cap=96)
    path = os.path.join(tmp_path, 'small.safetensors')
    checkpoint.save_engine(path, eng)
    eng2 = Qwen3Int8Engine.from_int8(path, 96)
    prompt = torch.randint(0, SMALL.vocab, (9,), generator=torch.Generator().manual_seed(5))
    toks = []
    for e in (eng, eng2):
        e.reset()
        logits = e.prefill(prompt).float().cpu()
        e.capture()
        seq = [int(e.token)]
        for _ in range(12):
            e.replay()
            seq.append(int(e.token))
        toks.append((logits, seq))
    assert torch.equal(toks[0][0], toks[1][0])
    assert toks[0][1] == toks[1][1]


def _tiny_transformers(attn=None):
    transformers = pytest.importorskip('transformers')
    torch.manual_seed(0)
    kw = {'attn_implementation': attn} if attn else {}
    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                                   max_position_embeddings=256, tie_word_embeddings=True, initializer_range=0.2, **kw)
    return transformers.Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


def test_graph_decoder_quantize_opt_in_matches_quantize_model():
    """A bf16 transformers model is refused without quantize=True (tested on the CPU); with it, the decoder's
    tokens equal those of the same model quantised by quantize_model first."""
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    from efficientgpt_amd.int8_linear import quantize_model
    a = _tiny_transformers().cuda()
    b = _tiny_transformers().cuda()
    quantize_model(b)
    x = torch.randint(0, 512, (1, 9), generator=torch.Generator().manual_seed(8)).cuda()
    got, _ = GraphGreedyDecoder(a, max_cache_len=64, quantize=True).generate(x, 30)
    want, _ = GraphGreedyDecoder(b, max_cache_len=64).generate(x, 30)
    assert got == want
    assert len(set(got)) > 8


def test_hf_adapter_batch_of_two_and_left_padding():
    """transformers generate() with attn_implementation 'egpt_decode': an unpadded batch of two equals each row
    decoded alone by eager SDPA attention within the near-tie rule; a left-padded batch raises ValueError (the
    kernel reads cache slots 0..position and cannot mask padding) instead of attending the pad slots."""
    transformers = pytest.importorskip('transformers')
    from efficientgpt_amd import hf
    hf.register()
    model = _tiny_transformers(hf.NAME).cuda()
    ref = _tiny_transformers('sdpa').cuda()
    x = torch.randint(0, 512, (2, 7), generator=torch.Generator().manual_seed(9)).cuda()
    kw = dict(max_new_tokens=16, min_new_tokens=16, do_sample=False, pad_token_id=0)
    with torch.no_grad():
        got = model.generate(input_ids=x, attention_mask=torch.ones_like(x), **kw)[:, 7:].tolist()
        for row in range(2):
            out = ref.generate(input_ids=x[row:row + 1], attention_mask=torch.ones_like(x[row:row + 1]),
                               output_scores=True, return_dict_in_generate=True, **kw)
            want = out.sequences[0, 7:].tolist()
            if got[row] != want:  # free-running decodes may part at a near-tie of the two attention forms
                i = next(j for j, (p, q) in enumerate(zip(got[row], want)) if p != q)
                top = out.scores[i][0].float().topk(2).values
                assert float(top[0] - top[1]) < near_tie_bound(float(top[0])), (row, i)
        mask = torch.ones_like(x)
        mask[0, :2] = 0
        with pytest.raises(ValueError, match='padd'):
            model.generate(input_ids=x, attention_mask=mask, **kw)
