"""The greedy pick follows torch.argmax: NaN ranks above every number (the first NaN wins), otherwise the largest
value, ties to the first index. Through the stand-alone egpt_argmax and through the decode step's lm_head GEMV,
whose argmax epilogue reduces per-block maxima (egpt_int8_gemv_fused + egpt_argmax_parts)."""

import ctypes

import pytest
import torch

from efficientgpt_amd import _lib

pytestmark = pytest.mark.gpu


def _argmax(logits):
    lib = _lib.lib()
    n = logits.numel()
    need = ctypes.c_size_t()
    _lib.check('egpt_argmax_workspace', lib.egpt_argmax_workspace(n, ctypes.byref(need)))
    ws = torch.empty(need.value, dtype=torch.uint8, device='cuda')
    token = torch.full((1,), -5, dtype=torch.long, device='cuda')
    position = torch.zeros(1, dtype=torch.long, device='cuda')
    _lib.check('egpt_argmax', lib.egpt_argmax(logits.data_ptr(), n, ws.data_ptr(), ws.numel(), token.data_ptr(),
                                              position.data_ptr(), _lib.stream_ptr()))
    torch.cuda.synchronize()
    assert int(position) == 1
    return int(token)


@pytest.mark.parametrize('case', ['plain', 'ties', 'nan', 'nan_and_inf', 'all_nan', 'all_neg_inf'])
def test_argmax_follows_torch(case):
    n = 151936
    x = torch.randn(n, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    if case == 'ties':
        x[[900, 77, 150000]] = 40.0
    elif case == 'nan':
        x[[90000, 70001, 140000]] = float('nan')
    elif case == 'nan_and_inf':
        x[10] = float('inf')
        x[[120000, 5000]] = float('nan')
    elif case == 'all_nan':
        x[:] = float('nan')
    elif case == 'all_neg_inf':
        x[:] = float('-inf')
    want = int(torch.argmax(x.float()))
    assert _argmax(x.cuda()) == want, case


def test_step_greedy_pick_with_nan_logits():
    """NaN scales on two lm_head rows make those logits NaN: the step picks the first of them, as torch.argmax
    of the step's own logits does."""
    from efficientgpt_amd.qwen3 import Qwen3Config, Qwen3Int8Engine
    cfg = Qwen3Config(vocab=4096, hidden=512, inter=1024, layers=2, heads=16, kv_heads=8, head_dim=128)
    eng = Qwen3Int8Engine.random(cfg, 64, seed=1, std=0.1)
    eng.reset()
    eng.prefill(torch.arange(5))
    eng.step()
    clean = int(eng.token)
    assert clean == int(torch.argmax(eng.logits[0].float()))
    eng.head_s[[3000, 1700]] = float('nan')
    eng.reset()
    eng.prefill(torch.arange(5))
    eng.step()
    torch.cuda.synchronize()
    assert bool(torch.isnan(eng.logits[0, 1700].float()))
    assert int(eng.token) == 1700 == int(torch.argmax(eng.logits[0].float()))
