"""The int8 on-disk format (efficientgpt_amd/checkpoint.py): a stored layout loads bit-identical, foreign or
mismatched files are refused, and packing float weights quantises exactly as the reference's quantize_weight."""

import os

import pytest
import torch

from efficientgpt_amd import checkpoint
from efficientgpt_amd.qwen3 import Qwen3Config, pack_qwen3
from oracle.qwen3 import TINY, quantize_weights, random_weights

CFG = Qwen3Config(TINY.vocab, TINY.hidden, TINY.inter, TINY.layers, TINY.heads, TINY.kv_heads, TINY.head_dim,
                  TINY.rope_theta, TINY.rms_eps, TINY.tied)


def packed_equal(a, b):
    if len(a['layers']) != len(b['layers']):
        return False
    for la, lb in zip(a['layers'], b['layers']):
        if la.keys() != lb.keys() or not all(la[k].dtype == lb[k].dtype and torch.equal(la[k], lb[k]) for k in la):
            return False
    return all(a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]) for k in ('embed', 'norm_w', 'head_q', 'head_s'))


def test_round_trip_is_bit_identical(tmp_path):
    pk = pack_qwen3(CFG, quantize_weights(random_weights(TINY, seed=1, std=0.2), TINY))
    inv = 1.0 / (1e4 ** (torch.arange(0, 32, 2).float() / 32))
    path = os.path.join(tmp_path, 'tiny.safetensors')
    checkpoint.save_int8(path, CFG, pk, inv_freq=inv)
    cfg, got, inv2 = checkpoint.load_int8(path)
    assert cfg == CFG
    assert packed_equal(pk, got)
    assert torch.equal(inv2, inv)


def test_float_weights_pack_like_quantised_ones():
    """Given float linears, pack_qwen3 quantises them (int8_linear.py:106-117); the result equals packing the
    oracle's own quantisation of the same weights, tied head included."""
    w = random_weights(TINY, seed=2, std=0.2)
    assert packed_equal(pack_qwen3(CFG, w), pack_qwen3(CFG, quantize_weights(w, TINY)))


def test_foreign_and_mismatched_files_are_refused(tmp_path):
    from safetensors.torch import save_file
    other = os.path.join(tmp_path, 'other.safetensors')
    save_file({'x': torch.zeros(2)}, other, metadata={'format': 'pt'})
    with pytest.raises(ValueError, match='not an'):
        checkpoint.load_int8(other)
    pk = pack_qwen3(CFG, quantize_weights(random_weights(TINY, seed=3, std=0.2), TINY))
    pk['layers'][1]['o_q'] = pk['layers'][1]['o_q'][:, :-16].contiguous()
    bad = os.path.join(tmp_path, 'bad.safetensors')
    checkpoint.save_int8(bad, CFG, pk)
    with pytest.raises(ValueError, match='layer 1 o_q'):
        checkpoint.load_int8(bad)


@pytest.mark.parametrize('key,cut', [('q_norm', 'qn_w'), ('post_norm', 'post_w'), ('final', None), ('head_s', None),
                                     ('embed_dtype', None)])
def test_every_stored_tensor_is_checked(tmp_path, key, cut):
    """Norm vectors, the final norm, the head's scales and the embedding's dtype are checked against the config
    too, so a short or mistyped tensor never reaches a kernel."""
    pk = pack_qwen3(CFG, quantize_weights(random_weights(TINY, seed=4, std=0.2), TINY))
    if cut:
        pk['layers'][0][cut] = pk['layers'][0][cut][:-8].contiguous()
        match = f'layer 0 {cut}'
    elif key == 'final':
        pk['norm_w'] = pk['norm_w'][:-8].contiguous()
        match = 'final_norm'
    elif key == 'head_s':
        pk['head_s'] = pk['head_s'][:-1].contiguous()
        match = 'lm_head scale'
    else:
        pk['embed'] = pk['embed'].float()
        match = 'embed'
    bad = os.path.join(tmp_path, 'bad.safetensors')
    checkpoint.save_int8(bad, CFG, pk)
    with pytest.raises(ValueError, match=match):
        checkpoint.load_int8(bad)


@pytest.mark.parametrize('packed', [True, False])
def test_engine_refuses_weights_that_do_not_match_the_config(packed):
    """The engine checks the packed layout itself, whatever it was built from (packed tensors, or transformers-named
    weights through pack_qwen3): a short q_proj or o_proj raises before any tensor reaches the device."""
    from efficientgpt_amd.qwen3 import Qwen3Int8Engine
    w = quantize_weights(random_weights(TINY, seed=5, std=0.2), TINY)
    if packed:
        pk = pack_qwen3(CFG, w)
        pk['layers'][0]['o_q'] = pk['layers'][0]['o_q'][:, :-16].contiguous()
        arg, match = pk, 'layer 0 o_q'
    else:
        name = 'model.layers.1.self_attn.q_proj'
        w[name + '.qweight'] = w[name + '.qweight'][:-8].contiguous()
        w[name + '.scale'] = w[name + '.scale'][:-8].contiguous()
        arg, match = w, 'layer 1 qkv_q'
    with pytest.raises(ValueError, match=match):
        Qwen3Int8Engine(CFG, arg, 16, device='cpu', packed=packed)
