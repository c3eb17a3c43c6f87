"""Device-side int8 quantisation against the CPU oracle, bit for bit.

The reference runs its quantisation identity on the GPU (research/realmodel/
test_int8_linear.py:43-53, `device='cuda'`): quantize_weight on a 20000 x 64 matrix,
more than one 8192-row block, must give the whole-matrix formula's codes and steps
exactly. Here `quantize_weight` of a device tensor runs egpt_quantize_rows, and its
codes and steps are compared with oracle.int8.quantize_weight (numpy, pinned in
tests/test_oracle.py) at that case, at a bf16 12288 x 2048 gate/up matrix and at the
151936 x 2048 lm_head, plus rows built so that w / s lands exactly on .5 (round half
to even decides them), all-zero rows (the 1e-12 floor), fp16 and strided inputs.
`quantize_model` on a transformers model that lives on the GPU is then checked
against the oracle's codes of the same float weights, tied head included.
"""

import numpy as np
import pytest
import torch

from oracle import int8 as oint8

pytestmark = pytest.mark.gpu


def assert_same_as_oracle(w_dev, q, s, block=16384):
    """q / s (device) equal the oracle's on the same float values, bit for bit (rows in blocks, to bound the
    oracle's fp32 temporaries)."""
    wf = w_dev.float().cpu().numpy()
    qn, sn = q.cpu().numpy(), s.cpu().numpy()
    assert qn.dtype == np.int8 and sn.dtype == np.float32
    for r0 in range(0, wf.shape[0], block):
        wq, ws = oint8.quantize_weight(wf[r0:r0 + block])
        assert np.array_equal(ws.view(np.uint32), sn[r0:r0 + block].view(np.uint32)), r0
        assert np.array_equal(wq, qn[r0:r0 + block]), r0


def test_reference_case_20000x64_fp32():
    from efficientgpt_amd.int8_linear import quantize_weight
    torch.manual_seed(0)
    big = torch.randn(20000, 64, device='cuda')
    q, s = quantize_weight(big)
    assert q.device.type == 'cuda' and q.dtype == torch.int8 and s.dtype == torch.float32
    assert_same_as_oracle(big, q, s)
    # the reference's own assertion, on the device: the whole-matrix formula with no row blocks
    s_ref = (big.cpu().abs().amax(1) / 127.0).clamp_min(1e-12)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu(), torch.round(big.cpu() / s_ref[:, None]).clamp(-127, 127).to(torch.int8))
    # half-step reconstruction and the full code range (test_int8_linear.py:49-52)
    assert int(q.abs().amax(1).min()) == 127
    assert float((q.float() * s[:, None] - big).abs().max()) <= float(s.max()) / 2 + 1e-6


@pytest.mark.parametrize('n,k', [(12288, 2048), (151936, 2048)])
def test_bf16_model_shapes(n, k):
    from efficientgpt_amd.int8_linear import quantize_weight
    g = torch.Generator(device='cuda').manual_seed(n)
    w = (torch.randn(n, k, generator=g, device='cuda') * 0.02).to(torch.bfloat16)
    q, s = quantize_weight(w)
    assert_same_as_oracle(w, q, s)


def test_ties_zero_rows_fp16_and_strides():
    from efficientgpt_amd.int8_linear import quantize_weight
    # Rows whose max |w| is 127 * 2^e make s = 2^e exactly, so w = (j + 0.5) 2^e gives w / s = j + 0.5 exactly:
    # round half to even decides every element (2.5 -> 2, 3.5 -> 4, -0.5 -> -0, -126.5 -> -126).
    j = torch.arange(-127, 127, dtype=torch.float32) + 0.5
    rows = []
    for e in (-12, -7, 0, 3):
        r = torch.cat([j, torch.tensor([127.0, -127.0])]) * 2.0 ** e
        rows.append(r)
    ties = torch.stack(rows).cuda()
    q, s = quantize_weight(ties)
    assert torch.equal(s.cpu(), torch.tensor([2.0 ** e for e in (-12, -7, 0, 3)]))
    want = torch.round(j).clamp(-127, 127).to(torch.int8)  # torch.round is half to even
    assert torch.equal(q[:, :254].cpu(), want.expand(4, -1))
    assert_same_as_oracle(ties, q, s)
    # all-zero rows take the 1e-12 floor and code 0; a tiny row sits just above it
    z = torch.zeros(3, 100, device='cuda')
    z[2, 7] = 3e-10
    q, s = quantize_weight(z)
    assert_same_as_oracle(z, q, s)
    assert float(s[0]) == float(np.float32(1e-12)) and int(q[0].abs().max()) == 0
    # fp16 weights, and rows of a wider matrix (row stride > K) and a transposed view
    g = torch.Generator(device='cuda').manual_seed(7)
    h = (torch.randn(333, 96, generator=g, device='cuda') * 0.1).to(torch.float16)
    q, s = quantize_weight(h)
    assert_same_as_oracle(h, q, s)
    wide = torch.randn(257, 300, generator=g, device='cuda').to(torch.bfloat16)
    view = wide[:, 17:17 + 250]
    q, s = quantize_weight(view)
    assert_same_as_oracle(view, q, s)
    t = torch.randn(64, 200, generator=g, device='cuda').t()  # stride (1, 200): copied to rows first
    q, s = quantize_weight(t)
    assert_same_as_oracle(t, q, s)


def test_quantize_model_on_gpu_matches_oracle_codes():
    transformers = pytest.importorskip('transformers')
    from efficientgpt_amd.int8_linear import Int8Linear, quantize_model
    torch.manual_seed(0)
    cfg = transformers.Qwen3Config(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                                   max_position_embeddings=256, tie_word_embeddings=True, initializer_range=0.05)
    model = transformers.Qwen3ForCausalLM(cfg).to(torch.bfloat16).cuda().eval()
    floats = {n: m.weight.detach().clone() for n, m in model.named_modules() if isinstance(m, torch.nn.Linear)}
    embed = model.model.embed_tokens.weight.detach().clone()
    assert quantize_model(model) == len(floats)
    assert not model.config.tie_word_embeddings
    mods = dict(model.named_modules())
    for name, w in floats.items():
        m = mods[name]
        assert isinstance(m, Int8Linear) and m.qweight.is_cuda, name
        # the tied head's float weight is the embedding's: its codes are the embedding's
        assert_same_as_oracle(embed if name == 'lm_head' else w, m.qweight, m.scale)
    assert torch.equal(model.model.embed_tokens.weight, embed)  # the embedding keeps its bf16 weight
