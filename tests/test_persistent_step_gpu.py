"""The one-launch persistent decode step (egpt_qwen3_persistent_step) on Qwen3-1.7B widths.

Checked against the launch-per-phase fused step on the same inputs (teacher-forced: both
consume the same token at every step, so a near-tie cannot make them drift apart) and
against the CPU oracle (teacher-forced greedy agreement under the near-tie rule). The two steps differ only in
the attention's split structure (one split per kv head here, several in the fused
step), so logits agree to fp32-rounding-level differences carried through the bf16
activations: the tolerance is the 2e-2 relative bound of the north star.
"""

import pytest
import torch

from oracle.qwen3 import Qwen3Shape
from tests.test_qwen3_engine_gpu import WIDE2

pytestmark = pytest.mark.gpu

# Qwen3-1.7B widths at 6 layers and a small vocabulary (every per-layer phase, less memory)
WIDE6 = Qwen3Shape(vocab=4096, hidden=2048, inter=6144, layers=6, heads=16, kv_heads=8, head_dim=128)


def engine(shape, cap, seed, persistent=True):
    from efficientgpt_amd.qwen3 import Qwen3Config, Qwen3Int8Engine
    from oracle.qwen3 import quantize_weights, random_weights
    w = quantize_weights(random_weights(shape, seed=seed, std=0.05, norm_jitter=0.1), shape)
    cfg = Qwen3Config(shape.vocab, shape.hidden, shape.inter, shape.layers, shape.heads, shape.kv_heads,
                      shape.head_dim, shape.rope_theta, shape.rms_eps, shape.tied)
    return Qwen3Int8Engine(cfg, {k: v.cuda() for k, v in w.items()}, cap, persistent=persistent)


def forced_run(eng, fn, prompt, forced, n):
    eng.reset()
    eng.prefill(prompt)
    toks, logits = [], []
    for i in range(n):
        if forced is not None and i > 0:
            eng.token.fill_(forced[i - 1])
        fn()
        toks.append(int(eng.token))
        logits.append(eng.logits[0].float().cpu().clone())
    torch.cuda.synchronize()
    return toks, logits, eng.k_cache.float().cpu().clone(), eng.v_cache.float().cpu().clone(), int(eng.position)


def test_persistent_matches_oracle_teacher_forced():
    """Teacher-forced greedy steps of the persistent step against the CPU oracle (Qwen3-1.7B widths)."""
    from tests.test_qwen3_engine_gpu import oracle_greedy_with_margins, teacher_forced_agreement
    from efficientgpt_amd.qwen3 import Qwen3Config, Qwen3Int8Engine
    from oracle.qwen3 import Qwen3Oracle, quantize_weights, random_weights
    w = quantize_weights(random_weights(WIDE2, seed=21, std=0.05, norm_jitter=0.1), WIDE2)
    cfg = Qwen3Config(WIDE2.vocab, WIDE2.hidden, WIDE2.inter, WIDE2.layers, WIDE2.heads, WIDE2.kv_heads,
                      WIDE2.head_dim, WIDE2.rope_theta, WIDE2.rms_eps, WIDE2.tied)
    eng = Qwen3Int8Engine(cfg, {k: v.cuda() for k, v in w.items()}, 64, persistent=True)
    orc = Qwen3Oracle(WIDE2, w, dtype=torch.bfloat16, cap=64)
    prompt = torch.randint(0, WIDE2.vocab, (16,), generator=torch.Generator().manual_seed(5))
    ref, margins, tops = oracle_greedy_with_margins(orc, prompt, 12)
    assert len(set(ref)) > 4
    a, n, bad = teacher_forced_agreement(eng, prompt, ref, margins, tops)
    eng.check_status()
    assert not bad, bad
    assert a >= n - 1, (a, n)


@pytest.mark.parametrize('shape,cap,prompt_len', [(WIDE2, 64, 9), (WIDE6, 400, 300)])
def test_persistent_matches_fused_step(shape, cap, prompt_len):
    eng = engine(shape, cap, seed=11)
    prompt = torch.randint(0, shape.vocab, (prompt_len,), generator=torch.Generator().manual_seed(3))
    tf, lf, kf, vf, pf = forced_run(eng, eng.step_fused, prompt, None, 12)
    tp, lp, kp, vp, pp = forced_run(eng, eng.step_persistent, prompt, tf, 12)
    eng.check_status()
    assert pf == pp == prompt_len + 12
    for a, b in zip(lf, lp):
        assert float((a - b).abs().max()) <= 2e-2 * float(a.abs().max())
    assert torch.equal(vf[:, :, :prompt_len], vp[:, :, :prompt_len])  # prompt slots from the same prefill
    assert float((kf - kp).abs().max()) <= 2e-2 * float(kf.abs().max())
    assert float((vf - vp).abs().max()) <= 2e-2 * float(vf.abs().max())
    assert sum(a == b for a, b in zip(tf, tp)) >= 11, (tf, tp)


def test_persistent_graph_replay_equals_eager():
    """Same tokens and bit-identical logits from the captured graph and from eager launches."""
    eng = engine(WIDE2, 64, seed=5)
    prompt = torch.arange(7) * 13
    eng.reset()
    eng.prefill(prompt)
    eager, eager_logits = [], []
    for _ in range(10):
        eng.step()
        eager.append(int(eng.token))
        eager_logits.append(eng.logits[0].clone())
    eng.capture()
    eng.reset()
    eng.prefill(prompt)
    for i in range(10):
        eng.replay()
        assert int(eng.token) == eager[i]
        assert torch.equal(eng.logits[0], eager_logits[i])
    eng.check_status()


def test_persistent_through_tag_wraparound_and_long_context():
    """6100 steps of a 2-layer model: 11 hand-off phases per step, so the 16-bit row tags wrap
    (past 65536 phases) and the attention runs over up to 6108 slots in one split per kv head.
    The final step, teacher-forced, matches the fused step on the same cache."""
    eng = engine(WIDE2, 6144, seed=8)
    eng.reset()
    eng.prefill(torch.arange(8) * 7)
    eng.capture()
    for chunk in range(61):
        for _ in range(100):
            eng.replay()
        eng.check_status()  # synchronises: a failing step shows within 100 steps
    assert int(eng.position) == 8 + 6100
    tok, pos = int(eng.token), int(eng.position)
    k0, v0 = eng.k_cache.clone(), eng.v_cache.clone()
    out = {}
    for name, fn in (('fused', eng.step_fused), ('persistent', eng.step_persistent)):
        eng.token.fill_(tok)
        eng.position.fill_(pos)
        eng.k_cache.copy_(k0)
        eng.v_cache.copy_(v0)
        fn()
        out[name] = eng.logits[0].float().cpu().clone()
    eng.check_status()
    a, b = out['fused'], out['persistent']
    assert float((a - b).abs().max()) <= 2e-2 * float(a.abs().max())
