"""egpt_decode_attn_noalloc: the allocation-free form of egpt_decode_attn, through the C ABI.

Its split partials live in the library's per-device scratch array instead of a
caller's workspace; the kernels are the same, so its output must equal
egpt_decode_attn's bit for bit. Two calls in a row, the second with a smaller
input (fewer rows and splits: stale partials of the first call sit in the array
and must not leak into the second), then a graph that captures the call and is
replayed with eager work in between, each replay checked against the eager result.
"""

import ctypes

import numpy as np
import pytest
import torch

from efficientgpt_amd import _lib
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _inputs(b, hq, hkv, cap, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, 1, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16)
    v = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, cap, (b,), generator=g)
    pos[0] = cap - 1
    return q, k, v, pos


def _attend(q, k, v, pos, nsplit, workspace):
    """One call of egpt_decode_attn (workspace tensor) or egpt_decode_attn_noalloc (workspace None)."""
    lib = _lib.lib()
    b, hq, _, d = q.shape
    hkv, cap = k.shape[1], k.shape[2]
    out = torch.empty_like(q)
    head = [_lib.EGPT_BF16, q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
            pos.data_ptr(), 1, out.data_ptr(), out.stride(0), out.stride(1)]
    tail = [b, hq, hkv, cap, d, nsplit, d ** -0.5, _lib.stream_ptr()]
    if workspace is None:
        st = lib.egpt_decode_attn_noalloc(*head, *tail)
        _lib.check('egpt_decode_attn_noalloc', st)
    else:
        _lib.check('egpt_decode_attn', lib.egpt_decode_attn(*head, workspace.data_ptr(), workspace.numel(), *tail))
    return out


def _workspace(b, hq, hkv, cap, d, nsplit):
    need = ctypes.c_size_t()
    _lib.check('egpt_decode_attn_workspace', _lib.lib().egpt_decode_attn_workspace(b, hq, hkv, cap, d, nsplit,
                                                                                   ctypes.byref(need)))
    return torch.empty(need.value, dtype=torch.uint8, device='cuda')


def test_noalloc_equals_workspace_entry_point_on_two_calls_second_smaller():
    cases = [(4, 16, 8, 4096, 128, 0), (1, 16, 8, 700, 128, 0), (1, 32, 8, 2048, 128, 7), (2, 16, 8, 200, 128, 1)]
    for b, hq, hkv, cap, d, nsplit in cases:
        q, k, v, pos = (t.cuda() for t in _inputs(b, hq, hkv, cap, d, seed=cap))
        want = _attend(q, k, v, pos, nsplit, _workspace(b, hq, hkv, cap, d, nsplit))
        got = _attend(q, k, v, pos, nsplit, None)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (b, hq, hkv, cap, nsplit)
        truth = oatt.attention_truth(q.double().cpu().numpy(), k.double().cpu().numpy(), v.double().cpu().numpy(),
                                     pos.cpu().numpy())
        err = float(np.abs(got.double().cpu().numpy() - truth).max())
        assert err <= 2e-2 * float(np.abs(truth).max()), (b, hq, cap, err)


def test_noalloc_refuses_more_partials_than_its_scratch():
    q, k, v, pos = (t.cuda() for t in _inputs(1, 16, 8, 4096, 128, seed=1))
    lib = _lib.lib()
    out = torch.empty_like(q)
    args = [_lib.EGPT_BF16, q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), pos.data_ptr(), 1, out.data_ptr(),
            out.stride(0), out.stride(1)]
    assert lib.egpt_decode_attn_noalloc(*args, 1, 16, 8, 4096, 128, 505, 128 ** -0.5, _lib.stream_ptr()) == \
        _lib.EGPT_ERR_WORKSPACE
    assert lib.egpt_decode_attn_noalloc(*args, 1, 16, 8, 4096, 128, 504, 128 ** -0.5, _lib.stream_ptr()) == 0
    torch.cuda.synchronize()


def test_noalloc_under_graph_capture_replays_match_eager():
    b, hq, hkv, cap, d = 1, 16, 8, 2048, 128
    q, k, v, pos = (t.cuda() for t in _inputs(b, hq, hkv, cap, d, seed=5))
    eager = _attend(q, k, v, pos, 0, None)  # first call on the device: looks up the scratch address
    torch.cuda.synchronize()
    out = torch.empty_like(q)
    lib = _lib.lib()

    def call():
        _lib.check('egpt_decode_attn_noalloc', lib.egpt_decode_attn_noalloc(
            _lib.EGPT_BF16, q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), pos.data_ptr(), 1, out.data_ptr(),
            out.stride(0), out.stride(1), b, hq, hkv, cap, d, 0, d ** -0.5, _lib.stream_ptr()))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    other = _inputs(2, 16, 8, 4096, 128, seed=9)
    other = [t.cuda() for t in other]
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _attend(*other, 0, None)  # eager work on the same scratch between replays
        torch.cuda.synchronize()
