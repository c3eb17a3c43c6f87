"""Weight-only int8 linear layers backed by the gfx950 GEMV kernel.

Drop-in for research/realmodel/int8_linear.py: same op name and schema
(`efficientgpt::int8_linear(x, w, s) -> Tensor`, functional, with a fake
implementation), same `int8_matmul`, `quantize_weight`, `Int8Linear` and
`quantize_model` signatures, buffer names and error messages.

Weights are quantised per output channel, symmetric: s = max|w| / 127,
q = round(w / s) in [-127, 127] (round half to even); device tensors are quantised by
the HIP kernel egpt_quantize_rows (correctly rounded fp32 steps, the same bits as the
formula on the CPU). Decode (<= 16 rows) runs the HIP GEMV through libegpt_hip.so:
fp32 accumulation, scale applied to the finished sum, one bf16 rounding. Prefill
(> 16 rows) computes the reference's formula `((x @ q.bf16.T).float() * s).bf16`
(int8_linear.py:96-97) on the MFMA GEMM egpt_int8_gemm, which reads the int8 codes
directly (no bf16 copy of the weights).

`CONFIGS` / `DEFAULT` keep the reference's tuple format
(family, BLOCK_N, BLOCK_K, SPLITK, warps) (int8_linear.py:18-23): family
'dot16' is the single-pass kernel, 'dot16_splitk' the split-K pair with SPLITK
splits. BLOCK_N, BLOCK_K and warps are tile sizes of the reference's Triton
kernels; the HIP kernels pick their wavefront tiling from the shape, so those
three fields are accepted and ignored.
"""

import ctypes

import torch
from torch import nn

from . import _lib

MAX_DECODE_ROWS = 16
CONFIGS = {}
DEFAULT = ('dot16', 32, 128, 0, 4)
_FAMILIES = ('dot16', 'dot16_splitk')


def _check_operands(x2, w, s):
    if not (x2.is_cuda and w.is_cuda and s.is_cuda):
        raise ValueError('int8_linear runs on a ROCm GPU: x, w and s must be device tensors')
    if w.dtype != torch.int8 or w.dim() != 2:
        raise ValueError('int8_linear expects int8 weights [N, K]')
    if s.dtype != torch.float32 or s.shape != (w.shape[0],):
        raise ValueError('int8_linear expects fp32 scales [N]')
    if x2.shape[1] != w.shape[1]:
        raise ValueError(f'int8_linear: x has K={x2.shape[1]}, w has K={w.shape[1]}')


def int8_matmul(x2, w, s):
    """x2 bf16 [M <= 16, K] contiguous rows; w int8 [N, K]; s fp32 [N] -> bf16 [M, N]."""
    m, k = x2.shape
    n = w.shape[0]
    if m > MAX_DECODE_ROWS:  # more rows than the kernel's tile would leave output rows unwritten
        raise ValueError(f'int8_matmul handles at most {MAX_DECODE_ROWS} rows, got {m}')
    _check_operands(x2, w, s)
    if w.stride(1) != 1:
        w = w.contiguous()
    s = s.contiguous()
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    family, _bn, _bk, splitk, _warps = CONFIGS.get((k, n), DEFAULT)
    if family not in _FAMILIES:
        raise ValueError(f'unknown int8 GEMV family {family!r}')
    out = torch.empty((m, n), device=x2.device, dtype=torch.bfloat16)
    if m == 0 or n == 0:
        return out
    lib = _lib.lib()
    stream = _lib.stream_ptr(x2.device)
    if family == 'dot16' or splitk <= 1:
        st = lib.egpt_int8_gemv(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), s.data_ptr(),
                                out.data_ptr(), out.stride(0), m, n, k, stream)
        _lib.check('egpt_int8_gemv', st)
        return out
    need = ctypes.c_size_t()
    _lib.check('egpt_int8_gemv_splitk_workspace', lib.egpt_int8_gemv_splitk_workspace(m, n, k, splitk, need))
    part = torch.empty(max(need.value, 4), device=x2.device, dtype=torch.uint8)
    st = lib.egpt_int8_gemv_splitk(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), s.data_ptr(),
                                   out.data_ptr(), out.stride(0), m, n, k, splitk, part.data_ptr(), part.numel(),
                                   stream)
    _lib.check('egpt_int8_gemv_splitk', st)
    return out


@torch.library.custom_op('efficientgpt::int8_linear', mutates_args=())
def int8_linear(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.bfloat16:
        raise ValueError('int8_linear expects bf16 activations')
    if x2.shape[0] <= MAX_DECODE_ROWS:
        y = int8_matmul(x2.contiguous(), w, s)
    else:  # prefill: the reference's GEMM formula
        _check_operands(x2, w, s)
        y = int8_gemm(x2, w, s)
    return y.reshape(*x.shape[:-1], w.shape[0])


def int8_gemm(x2, w, s, out=None, workspace=None):
    """Prefill rows: bf16(fp32(bf16(x2 @ w^T)) * s), the reference's formula for more than 16 rows
    (research/realmodel/int8_linear.py:96-97), on the MFMA kernel egpt_int8_gemm, which reads the int8 weights
    directly (no bf16 copy of them). Measured on the MI355X against the reference's dequantise-then-library-GEMM
    formula at the Qwen3-1.7B and Qwen3-8B shapes: 1.2-2.9x faster at 128 rows, 1.1-1.4x at 1024-2048, and at
    8192 rows 0.93-1.4x (faster on 14 of 16 shapes, the whole 8B layer 8% faster). Shapes the MFMA kernel does
    not take (K not a multiple of 64, unaligned rows, operands of 2 GiB or more) run the library's generic kernel,
    the same formula without MFMA."""
    m, k = x2.shape
    n = w.shape[0]
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    if w.stride(1) != 1:
        w = w.contiguous()
    s = s.contiguous()
    if out is None:
        out = torch.empty((m, n), device=x2.device, dtype=torch.bfloat16)
    lib = _lib.lib()
    need = ctypes.c_size_t()
    _lib.check('egpt_int8_gemm_workspace', lib.egpt_int8_gemm_workspace(m, n, k, ctypes.byref(need)))
    ws = None
    if need.value:  # split K: the caller's workspace when it is large enough, else one from torch's allocator
        ws = workspace if workspace is not None and workspace.numel() >= need.value else \
            torch.empty(need.value, device=x2.device, dtype=torch.uint8)
    st = lib.egpt_int8_gemm_ws(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), s.data_ptr(),
                               out.data_ptr(), out.stride(0), m, n, k, ws.data_ptr() if ws is not None else None,
                               ws.numel() if ws is not None else 0, _lib.stream_ptr(x2.device))
    _lib.check('egpt_int8_gemm', st)
    return out


@int8_linear.register_fake
def _(x, w, s):
    return x.new_empty(*x.shape[:-1], w.shape[0])


ROW_BLOCK = 8192  # rows per quantisation block: bounds the fp32 temporaries of a 151,936-row head


def _quantize_rows(rows):
    """One block of rows (any float dtype) -> (int8 codes, fp32 per-row steps)."""
    wf = rows.float()
    step = torch.clamp_min(wf.abs().amax(dim=1) / 127.0, 1e-12)
    codes = torch.clamp(torch.round(wf / step.unsqueeze(1)), -127, 127).to(torch.int8)
    return codes, step


_QUANT_DTYPES = {torch.float32: _lib.EGPT_F32, torch.bfloat16: _lib.EGPT_BF16, torch.float16: _lib.EGPT_F16}


def _quantize_on_device(w):
    """(q, s) of a 2-D device tensor by egpt_quantize_rows: one launch, rows of any stride along dim 0."""
    if w.dtype not in _QUANT_DTYPES:
        w = w.float()  # the reference's `.float()` of the weight
    if w.dim() != 2 or w.shape[1] < 1:
        raise ValueError(f'quantize_weight expects a 2-D weight with K >= 1, got {tuple(w.shape)}')
    if w.stride(1) != 1:
        w = w.contiguous()
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s = torch.empty(n, dtype=torch.float32, device=w.device)
    st = _lib.lib().egpt_quantize_rows(_QUANT_DTYPES[w.dtype], w.data_ptr(), w.stride(0), n, k, q.data_ptr(),
                                       q.stride(0), s.data_ptr(), _lib.stream_ptr(w.device))
    _lib.check('egpt_quantize_rows', st)
    return q, s


def quantize_weight(weight):
    """Per-output-channel symmetric int8: returns (q int8 [N, K], s fp32 [N]) with weight ~= q * s[:, None].

    s = max(max_k |w| / 127, 1e-12) in fp32 and q = clamp(round(w / s), -127, 127)
    with round half to even (research/realmodel/int8_linear.py:106-117). Device tensors go
    through the HIP kernel egpt_quantize_rows, whose every step is one correctly rounded
    fp32 operation. Host tensors take the formula in torch; every row is independent, so
    quantising ROW_BLOCK rows at a time gives the same bits as the whole matrix at once.
    """
    w = weight.detach()
    if w.is_cuda:
        return _quantize_on_device(w)
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    s = torch.empty(w.shape[0], dtype=torch.float32, device=w.device)
    for lo in range(0, w.shape[0], ROW_BLOCK):
        hi = min(lo + ROW_BLOCK, w.shape[0])
        q[lo:hi], s[lo:hi] = _quantize_rows(w[lo:hi])
    return q, s


class Int8Linear(nn.Module):
    """nn.Linear replacement holding `qweight` (int8 [N, K]), `scale` (fp32 [N]) and an optional frozen bias."""

    def __init__(self, linear):
        super().__init__()
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        qweight, scale = quantize_weight(linear.weight)
        self.register_buffer('qweight', qweight)
        self.register_buffer('scale', scale)
        bias = linear.bias
        self.bias = nn.Parameter(bias.detach().clone(), requires_grad=False) if bias is not None else None

    def forward(self, x):
        out = int8_linear(x, self.qweight, self.scale)
        if self.bias is not None:
            out = out + self.bias
        return out

    def extra_repr(self):
        return f'in={self.in_features}, out={self.out_features}, int8 per-channel'


def _release_cached_blocks():
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


@torch.no_grad()
def quantize_model(model, include_lm_head=True):
    """Swap every nn.Linear (the lm_head too unless include_lm_head=False) for Int8Linear in place; return the count.

    Embeddings and norms stay bf16. A tied lm_head becomes an untied int8 copy while
    the embedding keeps its bf16 weight, so the config is marked untied. Modules are
    looked up by name and each bf16 Linear is released right after its swap, so the
    load peak stays near the bf16 model plus one layer.
    """
    targets = []
    for name, module in model.named_modules():
        if isinstance(module, nn.Linear) and (include_lm_head or name != 'lm_head'):
            targets.append(name)
    for i, name in enumerate(targets, 1):
        owner_name, _, attr = name.rpartition('.')
        owner = model.get_submodule(owner_name) if owner_name else model
        setattr(owner, attr, Int8Linear(getattr(owner, attr)))
        if i % 16 == 0:
            _release_cached_blocks()
    if include_lm_head and hasattr(model, 'config'):
        model.config.tie_word_embeddings = False
    _release_cached_blocks()
    return len(targets)
