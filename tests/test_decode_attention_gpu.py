"""HIP split-K GQA decode attention vs the fp64 oracle.

Mirrors research/phase5/test_graph_gpu.py:205-261 and :302-398 (fp32 / bf16 / fp16
inputs, positions {0, cap-1, cap/2, random per row}, x8 scaled logits, NaN-poisoned
slots past the position, non-contiguous K/V, dispatch) and extends them to grouped
query heads at the Qwen3 shapes (16 query / 8 kv heads, D = 128, L up to 32768).
Bounds: no worse than 2x the error against fp64 of the same-dtype masked SDPA (run on
the CPU) or of the reference's own split-K algorithm in fp32 (the oracle's
restatement of research/phase5/decode_attention.py:31-71), with the reference's
floors (1e-6 fp32, 1e-3 bf16/fp16), and within 2e-2 relative everywhere. The second
yardstick is the reference's own practice (research/phase5/test_graph_gpu.py:305-307
bounds by 1.25x its accepted split-K kernel) for cases where SDPA is unusually accurate.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def sdpa_err_cpu(q, k, v, pos, truth):
    """max |SDPA(same dtype, CPU) - truth|: the reference's yardstick (K/V repeated per group)."""
    g = q.shape[1] // k.shape[1]
    kk, vv = k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
    cap = k.shape[2]
    allowed = torch.arange(cap).view(1, 1, 1, cap) <= pos.cpu().view(-1, 1, 1, 1)
    if q.dtype == torch.float32:
        out = F.scaled_dot_product_attention(q, kk, vv, attn_mask=allowed)
    else:  # low precision SDPA on the CPU computes through fp32; round the result like the dtype
        out = F.scaled_dot_product_attention(q.float(), kk.float(), vv.float(), attn_mask=allowed).to(q.dtype)
    return float((out.double().numpy() - truth).__abs__().max())


def splitk_err(q, k, v, pos, truth):
    """max |reference split-K algorithm in fp32 - truth| (K/V in the input dtype, math in fp32)."""
    got = oatt.attention_splitk(q.float().numpy(), k.float().numpy(), v.float().numpy(), pos.numpy())
    return float(np.abs(got.astype(np.float64) - truth).max())


def run_case(b, hq, hkv, cap, d, dtype, pos, scale=1.0, seed=0, floor=None, config=None, fn=None):
    from efficientgpt_amd.decode_attention import decode_attention
    if fn is None:
        fn = (lambda q, k, v, p: decode_attention(q, k, v, p, config=config))
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, 1, d, generator=g) * scale).to(dtype)
    k = (torch.randn(b, hkv, cap, d, generator=g) * scale).to(dtype)
    v = torch.randn(b, hkv, cap, d, generator=g).to(dtype)
    pos = torch.as_tensor(pos, dtype=torch.long)
    truth = oatt.attention_truth(q.double().numpy(), k.double().numpy(), v.double().numpy(), pos.numpy())
    out = fn(q.cuda(), k.cuda(), v.cuda(), pos.cuda())
    assert out.dtype == dtype and out.shape == (b, hq, 1, d)
    err = float(np.abs(out.double().cpu().numpy() - truth).max())
    if floor is None:
        floor = 1e-6 if dtype == torch.float32 else 1e-3
    yard = sdpa_err_cpu(q, k, v, pos, truth)
    if dtype == torch.float32 and cap <= 512:
        yard = max(yard, splitk_err(q, k, v, pos, truth))
    bound = max(2 * yard, floor)
    assert err <= bound, (b, hq, hkv, cap, d, dtype, pos.tolist(), err, bound)
    assert err <= 2e-2 * max(float(np.abs(truth).max()), 1e-30)
    return out


@pytest.mark.parametrize('batch,cap', [(1, 80), (1, 256), (16, 128), (16, 256), (3, 37), (2, 2)])
@pytest.mark.parametrize('scale', [1.0, 8.0])
def test_mha_fp32_against_fp64(batch, cap, scale):
    for pos in ([0], [cap - 1], [cap // 2], torch.randint(0, cap, (batch,), generator=torch.Generator().manual_seed(batch)).tolist()):
        run_case(batch, 6, 6, cap, 64, torch.float32, pos, scale=scale, seed=cap)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
@pytest.mark.parametrize('batch,cap', [(1, 256), (16, 128), (3, 37)])
def test_mha_low_precision(dtype, batch, cap):
    pos = torch.randint(0, cap, (batch,), generator=torch.Generator().manual_seed(cap)).tolist()
    run_case(batch, 6, 6, cap, 64, dtype, pos, seed=batch)


@pytest.mark.parametrize('L', [256, 1024, 4096, 16384, 32768])
def test_qwen3_gqa_shapes_bf16(L):
    # 16 query heads over 8 kv heads, D = 128, attending to all L slots (position L - 1)
    run_case(1, 16, 8, L, 128, torch.bfloat16, [L - 1], seed=L)


@pytest.mark.parametrize('hq,hkv', [(32, 8), (8, 1), (4, 2)])
def test_other_groupings(hq, hkv):
    run_case(2, hq, hkv, 300, 128, torch.bfloat16, [5, 299], seed=hq)
    run_case(1, hq, hkv, 100, 64, torch.float32, [77], seed=hkv)


def test_split_count_invariance_and_single_pass():
    from efficientgpt_amd.decode_attention import decode_attention, decode_attention_single_pass
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 16, 1, 128, generator=g).cuda()
    k = torch.randn(1, 8, 2048, 128, generator=g).cuda()
    v = torch.randn(1, 8, 2048, 128, generator=g).cuda()
    pos = torch.tensor([1999], device='cuda')
    base = decode_attention_single_pass(q, k, v, pos)
    for split in (4, 16, 64, 256, 2048):  # 512, 128, 32, 8 and 1 splits
        other = decode_attention(q, k, v, pos, config=(split, 0, 0))
        assert float((other - base).abs().max()) < 1e-5


def test_never_reads_past_position():
    from efficientgpt_amd.decode_attention import decode_attention
    q = torch.randn(4, 16, 1, 128, device='cuda', dtype=torch.bfloat16)
    k = torch.randn(4, 8, 96, 128, device='cuda', dtype=torch.bfloat16)
    v = torch.randn_like(k)
    pos = torch.tensor([0, 17, 63, 94], device='cuda')
    clean = decode_attention(q, k, v, pos)
    for b, p in enumerate(pos.tolist()):
        k[b, :, p + 1:] = float('nan')
        v[b, :, p + 1:] = float('nan')
    assert torch.equal(clean, decode_attention(q, k, v, pos))


def test_strided_kv_and_mha_equivalence():
    from efficientgpt_amd.decode_attention import decode_attention
    q = torch.randn(4, 6, 1, 64, device='cuda')
    pos = torch.tensor([0, 17, 63, 94], device='cuda')
    kt = torch.randn(4, 96, 6, 64, device='cuda').transpose(1, 2)  # head-major view of [B, cap, H, D]
    vt = torch.randn(4, 96, 6, 64, device='cuda').transpose(1, 2)
    a = decode_attention(q, kt, vt, pos)
    b = decode_attention(q, kt.contiguous(), vt.contiguous(), pos)
    assert float((a - b).abs().max()) < 1e-5
    # GQA with Hkv = Hq / 2 equals MHA over K/V repeated per group
    k = torch.randn(2, 4, 50, 128, device='cuda', dtype=torch.bfloat16)
    v = torch.randn_like(k)
    q8 = torch.randn(2, 8, 1, 128, device='cuda', dtype=torch.bfloat16)
    p2 = torch.tensor([10, 49], device='cuda')
    gqa = decode_attention(q8, k, v, p2)
    mha = decode_attention(q8, k.repeat_interleave(2, 1).contiguous(), v.repeat_interleave(2, 1).contiguous(), p2)
    assert torch.equal(gqa, mha)


def test_validation_errors():
    from efficientgpt_amd.decode_attention import decode_attention
    q = torch.randn(1, 6, 1, 64, device='cuda')
    with pytest.raises(ValueError):
        decode_attention(q, q.half().expand(1, 6, 8, 64).contiguous(), q.expand(1, 6, 8, 64).contiguous(),
                         torch.tensor([3], device='cuda'))
    with pytest.raises(ValueError):
        decode_attention(q, q.expand(1, 6, 8, 64).contiguous(), q.expand(1, 6, 8, 64).contiguous(),
                         torch.tensor([3], device='cuda', dtype=torch.int32))
    with pytest.raises(ValueError):
        k = torch.randn(1, 4, 8, 64, device='cuda')
        decode_attention(q, k, k, torch.tensor([3], device='cuda'))  # 6 query heads over 4 kv heads


def test_graph_capture_follows_device_position():
    from efficientgpt_amd.decode_attention import decode_attention
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 16, 1, 128, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(1, 8, 512, 128, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(1, 8, 512, 128, generator=g).to(torch.bfloat16).cuda()
    pos = torch.tensor([0], device='cuda')
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        decode_attention(q, k, v, pos)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = decode_attention(q, k, v, pos)
    for p in (0, 5, 130, 511, 64):
        pos.fill_(p)
        graph.replay()
        eager = decode_attention(q, k, v, torch.tensor([p], device='cuda'))
        torch.cuda.synchronize()
        assert torch.equal(out, eager), p


@pytest.mark.parametrize('b,hq,hkv,cap', [
    (32, 16, 8, 1024),   # 256 (row, kv head) programs: single pass
    (31, 16, 8, 1024),   # 248 programs, 1024 slots: split-K
    (1, 16, 8, 256),     # few programs, 256 slots: single pass
    (1, 16, 8, 257),     # few programs, 257 slots: split-K
    (16, 6, 6, 256),     # the reference's Phase-5 MHA shape at its cache size
    (64, 6, 6, 1024),    # 384 programs: single pass
])
def test_dispatch_both_sides_of_its_thresholds(b, hq, hkv, cap):
    """decode_attention_dispatch (research/phase5/decode_attention.py:157-169; its tests test_graph_gpu.py:400-405)
    picks single pass exactly where use_single_pass says, and each choice meets the oracle's bounds. Its output
    is bit-identical to the form it chose."""
    from efficientgpt_amd.decode_attention import (decode_attention, decode_attention_dispatch,
                                                   decode_attention_single_pass, use_single_pass)
    d = 128 if hq != 6 else 64
    pos = torch.randint(0, cap, (b,), generator=torch.Generator().manual_seed(b + cap))
    pos[0] = cap - 1
    out = run_case(b, hq, hkv, cap, d, torch.bfloat16, pos, seed=3, fn=decode_attention_dispatch)
    single = use_single_pass(b, hkv, cap)
    assert single == (b * hkv >= 256 or cap <= 256)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(b, hq, 1, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16).cuda()
    chosen = decode_attention_single_pass if single else decode_attention
    assert torch.equal(out, chosen(q, k, v, pos.cuda()))
