"""Split-K GQA decode attention (one query per row and head) on the gfx950 kernels.

Drop-in for research/phase5/decode_attention.py: `decode_attention(q, k, v,
position, config=None)`, `decode_attention_single_pass`, `default_config`,
`use_single_pass` and `decode_attention_dispatch` keep the reference's names,
argument meaning and ValueError messages. The contract is widened to grouped
query attention: k/v may carry fewer heads than q (`k/v [B, Hkv, cap, D]`,
Hq % Hkv == 0, query head h reads kv head h // (Hq // Hkv)); with Hkv == Hq it is
the reference's multi-head contract.

Semantics: masked attention over slots <= position[b] with scale 1/sqrt(D), fp32
math, output stored in the input dtype. Slots past the position are never read,
and the position is read on the device, so the call can be captured in a graph.
Different fp32 summation order than masked SDPA: not bit-exact against it.
"""

import ctypes

import torch

from . import _lib

_SUPPORTED_D = (32, 64, 128)
_SUPPORTED_GROUPS = (1, 2, 4, 8)


def default_config(batch, heads, capacity):
    """(SPLIT, BLOCK_N, num_warps) in the reference's format (decode_attention.py:74-78).

    SPLIT is the number of cache slots per split at full capacity; the HIP kernel
    re-cuts the live range into the same number of splits at run time. BLOCK_N and
    num_warps describe Triton tiles and are ignored by the HIP kernels.
    """
    nsplit = _lib.lib().egpt_decode_attn_default_splits(batch, heads, capacity)
    return -(-capacity // nsplit), 0, 0


def _validate(q, k, v, position):
    b, h, one, d = q.shape
    cap = k.size(2)
    if one != 1 or k.dim() != 4 or k.size(0) != b or k.size(3) != d or v.shape != k.shape:
        raise ValueError('decode_attention expects q [B,H,1,D] and k/v [B,H,cap,D]')
    hkv = k.size(1)
    if hkv < 1 or h % hkv != 0:
        raise ValueError('decode_attention expects q [B,H,1,D] and k/v [B,H,cap,D]')
    if q.dtype not in (torch.float32, torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError('q, k, v must share one dtype: float32, bfloat16 or float16')
    if position.dtype != torch.long or position.numel() not in (1, b):
        raise ValueError('position must be int64 with 1 or B elements')
    if d not in _SUPPORTED_D or h // hkv not in _SUPPORTED_GROUPS:
        raise ValueError(f'decode_attention supports D in {_SUPPORTED_D} and Hq/Hkv in {_SUPPORTED_GROUPS}')
    if not (q.is_cuda and k.is_cuda and v.is_cuda and position.is_cuda):
        raise ValueError('decode_attention runs on a ROCm GPU: q, k, v and position must be device tensors')
    return b, h, hkv, cap, d


def _aligned(t, dims):
    """Last dim contiguous and every stride in `dims` a multiple of 16 bytes (16-byte lane loads).

    A stride of 0 (a batch dimension expanded over one cache) is aligned.
    """
    esz = t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all((t.stride(i) * esz) % 16 == 0 for i in dims))


def _run(q, k, v, position, nsplit, scale=None):
    b, h, hkv, cap, d = _validate(q, k, v, position)
    if not _aligned(q, (0, 1)):
        q = q.contiguous()
    if not _aligned(k, (0, 1, 2)):
        k = k.contiguous()
    if not _aligned(v, (0, 1, 2)):
        v = v.contiguous()
    lib = _lib.lib()
    if nsplit <= 0:
        nsplit = lib.egpt_decode_attn_default_splits(b, hkv, cap)
    need = ctypes.c_size_t()
    _lib.check('egpt_decode_attn_workspace', lib.egpt_decode_attn_workspace(b, h, hkv, cap, d, nsplit, need))
    ws = torch.empty(need.value, device=q.device, dtype=torch.uint8)
    out = torch.empty((b, h, 1, d), device=q.device, dtype=q.dtype)  # fp32 math, stored in the input dtype
    pos_stride = 0 if position.numel() == 1 else position.stride(0)
    st = lib.egpt_decode_attn(_lib.dtype_code(q.dtype),
                              q.data_ptr(), q.stride(0), q.stride(1),
                              k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
                              v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
                              position.data_ptr(), pos_stride,
                              out.data_ptr(), out.stride(0), out.stride(1),
                              ws.data_ptr(), ws.numel(),
                              b, h, hkv, cap, d, nsplit, d ** -0.5 if scale is None else float(scale),
                              _lib.stream_ptr(q.device))
    _lib.check('egpt_decode_attn', st)
    return out


def decode_attention(q, k, v, position, config=None):
    """q [B, Hq, 1, D], k/v [B, Hkv, cap, D] (fp32/bf16/fp16, fp32 math); position int64 [1] or [B]:
    keys at slots <= position[b]. Split-K partials plus the partial-softmax reduce."""
    if config is None:
        nsplit = 0
    else:
        split = int(config[0])
        if split < 1:
            raise ValueError('config SPLIT must be >= 1')
        nsplit = -(-k.size(2) // split)
    return _run(q, k, v, position, nsplit)


def decode_attention_single_pass(q, k, v, position, block_n=64, warps=2):
    """Same contract as decode_attention, one split per (row, kv head): no cross-split reduce."""
    return _run(q, k, v, position, 1)


# Shape-only dispatch (positions live on the device inside a graph): single pass when
# there are enough (row, kv head) programs to fill the GPU or the cache is short.
# Mirrors research/phase5/decode_attention.py:157-169; the thresholds are this
# kernel's, from its dispatch grid on the MI355X (`bench.py --dispatch-grid`): up to
# 256 slots one pass is 1.0-1.8x faster, and from 256 programs on both forms time
# the same. They are where egpt_decode_attn_default_splits returns 1, so
# decode_attention() with no config makes the same choice.
SINGLE_PASS_MIN_PROGRAMS = 256
SINGLE_PASS_MAX_CAPACITY_FEW_PROGRAMS = 256


def use_single_pass(batch, heads, capacity):
    return batch * heads >= SINGLE_PASS_MIN_PROGRAMS or capacity <= SINGLE_PASS_MAX_CAPACITY_FEW_PROGRAMS


def decode_attention_dispatch(q, k, v, position):
    b = q.size(0)
    if use_single_pass(b, k.size(1), k.size(2)):
        return decode_attention_single_pass(q, k, v, position)
    return decode_attention(q, k, v, position)
