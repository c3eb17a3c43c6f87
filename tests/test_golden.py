"""The oracle against the committed golden fixtures (tests/golden/, from tests/golden/make_golden.py).

The fixtures' expected values come from formulas independent of oracle/: torch's CPU
matmul for the reference's int8 rule, the fp64 closed form x.double() @ (q.double()
* s).T, torch's fp64 scaled_dot_product_attention, and transformers' Qwen3 for the
greedy tokens. A mistake in the oracle's quantiser, row rule, masking or model
(a dropped term, a wrong index) moves its outputs off these values.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import int8 as oint8
from tests.golden_cases import attention_cases, bf16_to_f32, bf16_ulp, linear_cases, tiny_greedy
from tests.near_tie import near_tie_bound


def test_oracle_quantize_matches_golden():
    for c in linear_cases():
        q, s = oint8.quantize_weight(bf16_to_f32(c['w']))
        assert np.array_equal(q, c['q']), tuple(c['shape'])
        assert np.array_equal(s, c['s']), tuple(c['shape'])


def test_oracle_int8_linear_matches_golden():
    for c in linear_cases():
        shape = tuple(int(v) for v in c['shape'])
        x = bf16_to_f32(c['x'])
        got = oint8.linear(x, c['q'], c['s'])
        rule = bf16_to_f32(c['rule'])
        # the same roundings; fp32 sums taken in another order may move a result by one bf16 ulp
        assert np.all(np.abs(got - rule) <= bf16_ulp(rule)), shape
        assert np.mean(got == rule) >= 0.98, shape
        # one bf16 rounding of a (nearly) exact sum, two for the > 16-row GEMM form
        ulps = 1.0 if shape[0] <= 16 else 2.0
        assert np.all(np.abs(got - c['truth']) <= ulps * bf16_ulp(c['truth']) + 1e-6), shape


def test_oracle_attention_matches_golden():
    for c in attention_cases():
        q, k, v, pos = c['q'][:, :, None], c['k'], c['v'], c['pos']
        truth = c['truth']
        assert np.abs(oatt.attention_truth(q, k, v, pos)[:, :, 0] - truth).max() <= 1e-12
        split = oatt.attention_splitk(q, k, v, pos)[:, :, 0]
        assert np.abs(split - truth).max() <= 1e-5 * max(1.0, float(np.abs(truth).max()))


def teacher_forced(logits_fn, run):
    """Greedy steps with the fixture's own tokens fed back: (agreeing steps, non-near-tie disagreements)."""
    ref, margins, tops = run['tokens'], run['margins'], run['tops']
    got = [int(torch.argmax(logits_fn(run['prompt'], 0)))]
    pos = len(run['prompt'])
    for i in range(1, len(ref)):
        got.append(int(torch.argmax(logits_fn([ref[i - 1]], pos))))
        pos += 1
    bad = [i for i, (a, b) in enumerate(zip(ref, got)) if a != b and margins[i] >= near_tie_bound(tops[i])]
    return sum(a == b for a, b in zip(ref, got)), bad


def test_oracle_qwen3_tiny_matches_golden_tokens():
    pytest.importorskip('transformers')
    from oracle.qwen3 import Qwen3Oracle, Qwen3Shape
    from tests.golden.make_golden import quantized_state, state_sha256, tiny_model
    fx = tiny_greedy()
    model = tiny_model()
    state = quantized_state(model)
    assert state_sha256(state) == fx['weights_sha256'], 'tiny model weights drifted from the fixture'
    shape = Qwen3Shape(vocab=512, hidden=128, inter=256, layers=2, heads=4, kv_heads=2, head_dim=32,
                       rope_theta=fx['rope_theta'], rms_eps=fx['rms_eps'])
    orc = Qwen3Oracle(shape, state, dtype=torch.bfloat16, cap=128, inv_freq=model.model.rotary_emb.inv_freq)

    def logits(tokens, pos0):
        if pos0 == 0:
            orc.reset()
        return orc.forward(torch.tensor(tokens), pos0).float()

    for run in fx['runs']:
        assert len(set(run['tokens'])) > 8  # a degenerate model would make agreement trivial
        agree, bad = teacher_forced(logits, run)
        assert not bad, (len(run['prompt']), bad)
        assert agree >= 0.9 * len(run['tokens']), (len(run['prompt']), agree)
