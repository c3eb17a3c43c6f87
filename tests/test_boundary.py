"""Host-side behaviour of the drop-in boundary (CPU: nothing here launches a kernel).

- The op's fake implementation, which the reference pins through torch.compile parity
  (research/realmodel/test_int8_linear.py:62-79): under FakeTensorMode the op returns
  the reference's output shape and dtype for any leading dims, without running.
- GraphGreedyDecoder refuses a transformers model whose linears are still float: the
  decoder runs the int8 contract only (the reference's int8 backend quantises first,
  assistant/backends.py:200-202).
- The transformers attention adapter refuses positions and masks that are not a causal
  prefix of the cache (a left-padded batch) before any kernel runs.
"""

import pytest
import torch

from efficientgpt_amd import hf
from efficientgpt_amd.int8_linear import int8_linear


@pytest.mark.parametrize('lead', [(1,), (3,), (2, 5), (1, 1, 40)])
def test_int8_linear_fake_gives_output_shape_without_running(lead):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(*lead, 2048, dtype=torch.bfloat16)
        w = torch.empty(6144, 2048, dtype=torch.int8)
        s = torch.empty(6144, dtype=torch.float32)
        y = torch.ops.efficientgpt.int8_linear(x, w, s)
        assert tuple(y.shape) == (*lead, 6144)
        assert y.dtype == torch.bfloat16 and y.device == x.device
        y2 = int8_linear(x, w, s)  # the Python entry point dispatches to the same fake
        assert tuple(y2.shape) == (*lead, 6144)


def test_int8_linear_schema_is_the_reference_one():
    schema = torch.ops.efficientgpt.int8_linear.default._schema
    assert str(schema) == 'efficientgpt::int8_linear(Tensor x, Tensor w, Tensor s) -> Tensor'
    assert not schema.is_mutable


def _tiny_hf():
    transformers = pytest.importorskip('transformers')
    torch.manual_seed(0)
    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                                   max_position_embeddings=256, tie_word_embeddings=True, initializer_range=0.2)
    return transformers.Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


def test_graph_decoder_refuses_float_linears():
    from efficientgpt_amd.fast_decode import DecoderPool, GraphGreedyDecoder, engine_for
    model = _tiny_hf()
    with pytest.raises(ValueError, match='quantize_model'):
        GraphGreedyDecoder(model, max_cache_len=64)
    with pytest.raises(ValueError, match='quantize_model'):
        engine_for(model, 64)
    pool = DecoderPool(model, limit=256)
    with pytest.raises(ValueError, match='quantize_model'):
        pool.generate(torch.zeros((1, 4), dtype=torch.long), 4)


def test_graph_decoder_refuses_a_float_head():
    """quantize_model(model, include_lm_head=False) leaves the head in bf16, which the reference then runs in
    bf16; the engine's head is int8, so such a model is refused too."""
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    from efficientgpt_amd.int8_linear import quantize_model
    model = _tiny_hf()
    assert quantize_model(model, include_lm_head=False) == 14  # 7 linears x 2 layers, the head left float
    with pytest.raises(ValueError, match='first: lm_head'):
        GraphGreedyDecoder(model, max_cache_len=64)


def _qk(b, t, cap, hq=4, hkv=2, d=32):
    return torch.zeros(b, hq, t, d), torch.zeros(b, hkv, cap, d)


def test_hf_adapter_slots_for_unpadded_batches():
    q, k = _qk(2, 5, 16)
    pos = hf.query_slots(q, k, None, torch.arange(3, 8)[None])
    assert pos.tolist() == [[3, 4, 5, 6, 7]] * 2
    q, k = _qk(2, 1, 16)
    assert hf.query_slots(q, k, None, torch.tensor([[9], [9]])).tolist() == [[9], [9]]
    # no positions: the last T slots of the key tensor (a dynamic cache holds exactly the written slots)
    q, k = _qk(1, 3, 10)
    assert hf.query_slots(q, k).tolist() == [[7, 8, 9]]
    # a mask that is exactly the causal prefix is accepted, boolean or additive
    q, k = _qk(1, 2, 8)
    allowed = torch.arange(8)[None, None, None, :] <= torch.tensor([4, 5])[None, None, :, None]
    assert hf.query_slots(q, k, allowed, torch.tensor([[4, 5]])).tolist() == [[4, 5]]
    additive = torch.zeros(1, 1, 2, 8).masked_fill(~allowed, float('-inf'))
    assert hf.query_slots(q, k, additive, torch.tensor([[4, 5]])).tolist() == [[4, 5]]


def test_hf_adapter_refuses_padded_batches_and_foreign_masks():
    # left-padded prefill: transformers' position ids for a row with two pads
    q, k = _qk(2, 5, 16)
    with pytest.raises(ValueError, match='different positions'):
        hf.query_slots(q, k, None, torch.tensor([[0, 0, 0, 1, 2], [0, 1, 2, 3, 4]]))
    q, k = _qk(1, 5, 16)
    with pytest.raises(ValueError, match='consecutive'):
        hf.query_slots(q, k, None, torch.tensor([[0, 0, 0, 1, 2]]))
    # the decode steps of that batch: the rows write one cache slot but carry different positions
    q, k = _qk(2, 1, 16)
    with pytest.raises(ValueError, match='different positions'):
        hf.query_slots(q, k, None, torch.tensor([[3], [5]]))
    with pytest.raises(ValueError, match='outside the cache'):
        hf.query_slots(q, k, None, torch.tensor([[16], [16]]))
    # a mask hiding a slot before the query's own (padding), or showing one after it
    q, k = _qk(1, 1, 8)
    allowed = torch.arange(8)[None, None, None, :] <= 5
    hidden = allowed.clone()
    hidden[..., 1] = False
    with pytest.raises(ValueError, match='causal prefix'):
        hf.query_slots(q, k, hidden, torch.tensor([[5]]))
    with pytest.raises(ValueError, match='causal prefix'):
        hf.query_slots(q, k, allowed, torch.tensor([[4]]))


def test_hf_adapter_checks_each_position_tensor_once_and_rechecks_changes():
    """Every layer of a forward passes the same position_ids tensor: the host check runs for the first layer and is
    reused while that tensor is unchanged (no host read per layer); writing into it, or another mask, checks again."""
    q, k = _qk(1, 3, 16)
    pos = torch.arange(4, 7)[None]
    assert hf.query_slots(q, k, None, pos).tolist() == [[4, 5, 6]]
    ref, ver = hf._checked[0][0], hf._checked[0][1]
    assert ref() is pos and ver == pos._version
    assert hf._cached_positions(pos, None, (1, 3, 16)) is not None
    assert hf._cached_positions(pos.clone(), None, (1, 3, 16)) is None  # another tensor object: checked again
    assert hf._cached_positions(pos, None, (1, 3, 17)) is None  # another cache size
    allowed = torch.ones(1, 1, 3, 16, dtype=torch.bool)
    assert hf._cached_positions(pos, allowed, (1, 3, 16)) is None  # a mask that was not checked
    pos[0, 0] = 0  # written in place: its version moves, so the padded positions are caught
    with pytest.raises(ValueError, match='consecutive'):
        hf.query_slots(q, k, None, pos)


def test_prompt_attention_rule():
    """Which prompts take the causal prompt kernel: more than 64 rows whose last position reaches past 160; every
    other prompt runs the split-K decode kernel over its rows (host rule, no GPU)."""
    from efficientgpt_amd.qwen3 import use_prompt_kernel
    assert not use_prompt_kernel(64, 0) and not use_prompt_kernel(64, 8000)
    assert not use_prompt_kernel(128, 0) and not use_prompt_kernel(160, 0) and not use_prompt_kernel(100, 60)
    assert use_prompt_kernel(161, 0) and use_prompt_kernel(65, 96) and use_prompt_kernel(8192, 0)
