"""The HIP path against the committed golden fixtures (tests/golden/, from tests/golden/make_golden.py).

Same bars as the oracle's golden tests: the reference's int8 rule within one bf16
ulp and the fp64 truth within one (two for the > 16-row form); decode attention
against torch's fp64 SDPA; the fused decode step and the graph decoder against
transformers' greedy tokens on the reference's tiny Qwen3, disagreeing only at
near-ties (research/phase5/benchmark_review.py:46, 54-67).
"""

import numpy as np
import pytest
import torch

from tests.golden_cases import attention_cases, bf16_to_f32, bf16_ulp, linear_cases, tiny_greedy
from tests.near_tie import near_tie_bound, near_tie_match

pytestmark = pytest.mark.gpu


def test_int8_linear_matches_golden():
    from efficientgpt_amd.int8_linear import int8_linear
    for c in linear_cases():
        shape = tuple(int(v) for v in c['shape'])
        print('int8_linear golden', shape, flush=True)
        x = torch.from_numpy(c['x'].view(np.int16)).view(torch.bfloat16).cuda()
        q = torch.from_numpy(c['q']).cuda()
        s = torch.from_numpy(c['s']).cuda()
        got = int8_linear(x, q, s).float().cpu().numpy()
        rule = bf16_to_f32(c['rule'])
        assert np.all(np.abs(got - rule) <= bf16_ulp(rule)), shape
        assert np.mean(got == rule) >= 0.98, shape
        ulps = 1.0 if shape[0] <= 16 else 2.0
        assert np.all(np.abs(got - c['truth']) <= ulps * bf16_ulp(c['truth']) + 1e-6), shape


def test_decode_attention_matches_golden():
    from efficientgpt_amd.decode_attention import decode_attention
    for c in attention_cases():
        dt = torch.float32 if str(c['dtype']) == 'float32' else torch.bfloat16
        print('decode_attention golden', tuple(int(v) for v in c['shape']), dt, flush=True)
        q, k, v = (torch.from_numpy(c[n]).to(dt).cuda() for n in ('q', 'k', 'v'))
        pos = torch.from_numpy(c['pos']).cuda()
        for config in (None, (4, 0, 0)):  # default split count, and 4-slot splits
            got = decode_attention(q[:, :, None].contiguous(), k, v, pos, config=config)[:, :, 0].float().cpu().numpy()
            if dt == torch.float32:
                assert np.abs(got - c['truth']).max() <= 1e-5, config
            else:  # fp32 math, one bf16 rounding of the result
                assert np.all(np.abs(got - c['truth']) <= bf16_ulp(c['truth']) + 1e-5), config


@pytest.fixture(scope='module')
def tiny_engine():
    pytest.importorskip('transformers')
    from efficientgpt_amd.qwen3 import Qwen3Config, Qwen3Int8Engine
    from tests.golden.make_golden import quantized_state, state_sha256, tiny_model
    fx = tiny_greedy()
    model = tiny_model()
    state = quantized_state(model)
    assert state_sha256(state) == fx['weights_sha256'], 'tiny model weights drifted from the fixture'
    cfg = Qwen3Config(512, 128, 256, 2, 4, 2, 32, fx['rope_theta'], fx['rms_eps'], True)
    eng = Qwen3Int8Engine(cfg, {k: v.cuda() for k, v in state.items()}, 128,
                          inv_freq=model.model.rotary_emb.inv_freq)
    return eng, fx


def test_fused_step_matches_golden_tokens(tiny_engine):
    eng, fx = tiny_engine
    eng.capture()
    for run in fx['runs']:
        print('fused step golden, prompt', len(run['prompt']), flush=True)
        ref, margins, tops = run['tokens'], run['margins'], run['tops']
        eng.reset()
        eng.prefill(torch.tensor(run['prompt']))
        got = [int(eng.token)]
        for i in range(1, len(ref)):  # teacher-forced: the fixture's token is fed back
            eng.token.fill_(ref[i - 1])
            eng.replay()
            got.append(int(eng.token))
        bad = [i for i, (a, b) in enumerate(zip(ref, got)) if a != b and margins[i] >= near_tie_bound(tops[i])]
        assert not bad, (len(run['prompt']), bad)
        assert sum(a == b for a, b in zip(ref, got)) >= 0.9 * len(ref)


def test_graph_decoder_matches_golden_tokens(tiny_engine):
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    eng, fx = tiny_engine
    dec = GraphGreedyDecoder(eng, max_cache_len=128)
    for run in fx['runs']:
        print('graph decoder golden, prompt', len(run['prompt']), flush=True)
        got, st = dec.generate(torch.tensor([run['prompt']], device='cuda'), fx['new_tokens'])
        ok, i = near_tie_match(run['tokens'], got, run['margins'], run['tops'])
        assert ok, (len(run['prompt']), i)
        assert st['tokens'] == fx['new_tokens']
