"""HIP causal prompt-block attention (egpt_prefill_attn) vs the fp64 oracle.

The prompt pass of the reference's Qwen3 path is transformers' SDPA with a causal
mask over the static cache (HF models/qwen3/modeling_qwen3.py:252-280). On the
reference's GPU, bf16 SDPA runs the flash form, which rounds the probabilities to
bf16 before they multiply v; this kernel does the same. The error budget is
therefore that rounding plus the output's: with |dp| <= 2^-9 p per probability and
sum p / l = 1, |d out| <= 2^-9 max|v| + 2^-9 |out| <= 2^-8 max|v| (fp32 logits and
sums add far less). Each case must meet that bound and the 2e-2 relative bar.
Query heads per kv head 1, 2, 4 and 8 (and 3 and 6, which take blocks of 1 and 2
query heads); head dims 128, 64 and 32; prompts that start at slot 0 and ones that
continue a filled cache; strided rows; NaN in every slot past the block, which must
leave the output bit-identical; logits scaled x8; scores that climb along the prompt
and jump at a late slot, so the softmax's reference maximum moves many times.
"""

import numpy as np
import pytest
import torch

from efficientgpt_amd import _lib
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

D = 128


def _case(rows, hq, hkv, cap, pos0, seed, scale=1.0, q_pad=0, o_pad=0, D=D):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(rows, hq * D + q_pad, generator=g) * scale).to(torch.bfloat16)
    k = (torch.randn(hkv, cap, D, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(hkv, cap, D, generator=g).to(torch.bfloat16)
    return q, k, v, o_pad


def _run(q, k, v, hq, hkv, pos0, o_pad=0):
    rows, cap, D = q.shape[0], k.shape[1], k.shape[2]
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = torch.full((rows, hq * D + o_pad), 7.0, dtype=torch.bfloat16, device='cuda')
    st = _lib.lib().egpt_prefill_attn(qd.data_ptr(), qd.stride(0), kd.data_ptr(), vd.data_ptr(), kd.stride(0),
                                      kd.stride(1), out.data_ptr(), out.stride(0), rows, hq, hkv, D, cap, pos0,
                                      D ** -0.5, _lib.stream_ptr())
    _lib.check('egpt_prefill_attn', st)
    torch.cuda.synchronize()
    return out.cpu()


def _check(q, k, v, hq, hkv, pos0, o_pad=0):
    rows, D = q.shape[0], k.shape[2]
    out = _run(q, k, v, hq, hkv, pos0, o_pad)
    if o_pad:  # columns past the heads are never written
        assert torch.equal(out[:, hq * D:], torch.full((rows, o_pad), 7.0, dtype=torch.bfloat16))
    got = out[:, :hq * D].double().numpy().reshape(rows, hq, D)
    truth = oatt.prefill_truth(q[:, :hq * D].double().numpy().reshape(rows, hq, D), k.double().numpy(),
                               v.double().numpy(), pos0)
    err = float(np.abs(got - truth).max())
    bound = 2 ** -8 * float(v[:, :pos0 + rows].abs().max()) + 1e-4
    assert err <= bound, (rows, hq, hkv, pos0, err, bound)
    assert err <= 2e-2 * float(np.abs(truth).max())
    return out


@pytest.mark.parametrize('hq,hkv', [(8, 8), (16, 8), (32, 8), (64, 8)])
@pytest.mark.parametrize('rows,cap,pos0', [(67, 80, 0), (300, 320, 0), (130, 200, 37), (1, 16, 0), (129, 700, 500)])
def test_prefill_attention_matches_fp64(hq, hkv, rows, cap, pos0):
    q, k, v, _ = _case(rows, hq, hkv, cap, pos0, seed=rows + hq)
    _check(q, k, v, hq, hkv, pos0)


@pytest.mark.parametrize('d', [32, 64])
@pytest.mark.parametrize('hq,hkv', [(4, 2), (6, 6), (12, 4), (12, 2)])
@pytest.mark.parametrize('rows,cap,pos0', [(100, 128, 0), (130, 200, 37), (1, 16, 0)])
def test_prefill_attention_small_head_dims_and_any_group(d, hq, hkv, rows, cap, pos0):
    """Head dims 32 and 64 (the tiny test models and MHA 6 x 64), and groups of 3 and 6 query heads per kv head."""
    q, k, v, _ = _case(rows, hq, hkv, cap, pos0, seed=rows + hq + d, D=d)
    _check(q, k, v, hq, hkv, pos0)


@pytest.mark.parametrize('d', [32, 64])
def test_prefill_attention_small_head_dims_long_prompt(d):
    """Head dims 32 and 64 over a 1000-row prompt that continues 50 filled slots: 17 tiles for the last rows, so
    the tiles cycle many times through the kernel's K and V buffers at these dims' load counts."""
    q, k, v, _ = _case(1000, 8, 2, 1100, 50, seed=d + 7, D=d)
    _check(q, k, v, 8, 2, 50)


def test_prefill_attention_qwen3_8b_heads_long_prompt():
    # the Qwen3-8B grouping (32 / 8) over a 2048-token prompt: 32 tiles of 64 slots for the last rows
    q, k, v, _ = _case(2048, 32, 8, 2048, 0, seed=11)
    _check(q, k, v, 32, 8, 0)


@pytest.mark.parametrize('hq,hkv', [(16, 8), (32, 8)])
def test_prefill_attention_strided_rows_and_scaled_logits(hq, hkv):
    # q rows inside a wider buffer (the rotated queries of the fused QKV rows), output rows wider than the heads
    q, k, v, o_pad = _case(200, hq, hkv, 260, 40, seed=3, scale=8 ** 0.5, q_pad=2 * hkv * D, o_pad=64)
    _check(q, k, v, hq, hkv, 40, o_pad=o_pad)


@pytest.mark.parametrize('hq,hkv', [(16, 8), (32, 8)])
def test_prefill_attention_climbing_scores_and_a_late_spike(hq, hkv):
    # Non-negative queries against keys whose size climbs 60-fold along the slots: each query's maximum score
    # passes the softmax's reference maximum by more than 2^8 many times over the prompt; one key far larger
    # still (slot 700) makes it jump once more by hundreds of exponents, after which the rows attend almost only
    # to that slot. Every row must stay within the same bound of the fp64 truth.
    rows, cap = 1000, 1000
    g = torch.Generator().manual_seed(21)
    q = (torch.randn(rows, hq * D, generator=g).abs() * 0.5).to(torch.bfloat16)
    ramp = torch.linspace(0.2, 12.0, cap).view(1, cap, 1)
    kf = torch.randn(hkv, cap, D, generator=g).abs() * ramp
    kf[:, 700] = 40.0
    k = kf.to(torch.bfloat16)
    v = torch.randn(hkv, cap, D, generator=g).to(torch.bfloat16)
    _check(q, k, v, hq, hkv, 0)


@pytest.mark.parametrize('hq,hkv', [(16, 8), (32, 8)])
def test_prefill_attention_ignores_slots_past_the_block(hq, hkv):
    rows, cap, pos0 = 150, 400, 20
    q, k, v, _ = _case(rows, hq, hkv, cap, pos0, seed=5)
    clean = _run(q, k, v, hq, hkv, pos0)
    kp, vp = k.clone(), v.clone()
    kp[:, pos0 + rows:] = float('nan')
    vp[:, pos0 + rows:] = float('nan')
    assert torch.equal(_run(q, kp, vp, hq, hkv, pos0), clean)
    assert torch.equal(_run(q, k, v, hq, hkv, pos0), clean)  # reproducible run to run


def test_prefill_attention_refuses_what_it_does_not_take():
    lib = _lib.lib()
    q = torch.zeros(4, 16 * D, dtype=torch.bfloat16, device='cuda')
    kv = torch.zeros(8, 32, D, dtype=torch.bfloat16, device='cuda')
    out = torch.zeros_like(q)

    def call(rows=4, hq=16, hkv=8, d=D, cap=32, pos0=0):
        return lib.egpt_prefill_attn(q.data_ptr(), q.stride(0), kv.data_ptr(), kv.data_ptr(), kv.stride(0),
                                     kv.stride(1), out.data_ptr(), out.stride(0), rows, hq, hkv, d, cap, pos0,
                                     0.1, _lib.stream_ptr())
    assert call() == _lib.EGPT_OK
    assert call(d=96) == _lib.EGPT_ERR_UNSUPPORTED
    assert call(hq=12, hkv=8) < 0  # query heads not a multiple of the kv heads
    assert call(pos0=29) < 0 and call(pos0=29) != _lib.EGPT_ERR_UNSUPPORTED  # pos0 + rows past the cache
    assert call(rows=0) == _lib.EGPT_OK
    assert lib.egpt_prefill_attn(q.data_ptr(), q.stride(0), kv.data_ptr(), kv.data_ptr(), kv.stride(0), kv.stride(1),
                                 out.data_ptr(), out.stride(0), 4, 16, 8, D, 32, 0, -0.1, _lib.stream_ptr()) < 0
    torch.cuda.synchronize()
