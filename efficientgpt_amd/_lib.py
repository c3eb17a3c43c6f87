"""ctypes binding of libegpt_hip.so (the C ABI declared in include/egpt.h).

torch is imported first so the library binds to the HIP runtime torch already
loaded (both carry the SONAME libamdhip64.so.7): one runtime, one set of device
pointers and streams. There is no fallback: a missing or stale library raises.
"""

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / 'libegpt_hip.so'

EGPT_OK = 0
EGPT_ERR_UNSUPPORTED = -2
EGPT_ERR_WORKSPACE = -4
NOALLOC_SCRATCH_BYTES = 4 << 20  # EGPT_NOALLOC_SCRATCH_BYTES
EGPT_F32, EGPT_BF16, EGPT_F16 = 0, 1, 2
ABI_VERSION = 1

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_size = ctypes.c_size_t
_c_f = ctypes.c_float

# name -> (restype, argtypes); the full exported surface of include/egpt.h
SIGNATURES = {
    'egpt_abi_version': (_c_int, []),
    'egpt_status_string': (ctypes.c_char_p, [_c_int]),
    'egpt_int8_gemv': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp]),
    'egpt_quantize_rows': (_c_int, [_c_int, _c_vp, _c_i64, _c_int, _c_int, _c_vp, _c_i64, _c_vp, _c_vp]),
    'egpt_int8_gemm': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp]),
    'egpt_int8_gemm_workspace': (_c_int, [_c_int, _c_int, _c_int, ctypes.POINTER(_c_size)]),
    'egpt_int8_gemm_ws': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int,
                                   _c_vp, _c_size, _c_vp]),
    'egpt_int8_gemm_swiglu': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int,
                                       _c_vp]),
    'egpt_int8_gemm_add_rmsnorm': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64,
                                            _c_int, _c_int, _c_int, ctypes.c_float, _c_vp, _c_size, _c_vp]),
    'egpt_int8_gemm_qk_norm_rope': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                             _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _c_int, _c_f, _c_vp, _c_size, _c_vp]),
    'egpt_int8_gemv_splitk_workspace': (_c_int, [_c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_size)]),
    'egpt_int8_gemv_splitk': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_int,
                                       _c_int, _c_vp, _c_size, _c_vp]),
    'egpt_decode_attn_default_splits': (_c_int, [_c_int, _c_int, _c_int]),
    'egpt_qwen3_step_default_splits': (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    'egpt_decode_attn_workspace': (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_size)]),
    'egpt_decode_attn': (_c_int, [_c_int,
                                  _c_vp, _c_i64, _c_i64,
                                  _c_vp, _c_i64, _c_i64, _c_i64,
                                  _c_vp, _c_i64, _c_i64, _c_i64,
                                  _c_vp, _c_i64,
                                  _c_vp, _c_i64, _c_i64,
                                  _c_vp, _c_size,
                                  _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _c_vp]),
    'egpt_decode_attn_noalloc': (_c_int, [_c_int,
                                          _c_vp, _c_i64, _c_i64,
                                          _c_vp, _c_i64, _c_i64, _c_i64,
                                          _c_vp, _c_i64, _c_i64, _c_i64,
                                          _c_vp, _c_i64,
                                          _c_vp, _c_i64, _c_i64,
                                          _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _c_vp]),
    'egpt_rmsnorm': (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_f, _c_vp]),
    'egpt_add_rmsnorm': (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_f, _c_vp]),
    'egpt_qk_norm_rope': (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp,
                                   _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _c_vp]),
    'egpt_prefill_attn': (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_int, _c_int, _c_int,
                                   _c_int, _c_int, _c_int, _c_f, _c_vp]),
    'egpt_silu_mul': (_c_int, [_c_vp, _c_i64, _c_int, _c_vp, _c_i64, _c_int, _c_vp]),
    'egpt_embed': (_c_int, [_c_vp, _c_int, _c_vp, _c_i64, _c_int, _c_vp, _c_i64, _c_int, _c_vp]),
    'egpt_argmax_workspace': (_c_int, [_c_int, ctypes.POINTER(_c_size)]),
    'egpt_argmax': (_c_int, [_c_vp, _c_int, _c_vp, _c_size, _c_vp, _c_vp, _c_vp]),
    'egpt_qwen3_step_workspace': (_c_int, [_c_vp, ctypes.POINTER(_c_size)]),
    'egpt_qwen3_decode_step': (_c_int, [_c_vp, _c_vp]),
    'egpt_qwen3_step_gemvs': (_c_int, [_c_vp, _c_vp, _c_int, ctypes.POINTER(_c_int)]),
    'egpt_int8_gemv_fused_parts': (_c_int, [_c_vp, ctypes.POINTER(_c_int)]),
    'egpt_int8_gemv_fused': (_c_int, [_c_vp, _c_vp]),
    'egpt_argmax_parts': (_c_int, [_c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_vp]),
}

EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU, EPI_ARGMAX = 0, 1, 2, 3


class GemvFused(ctypes.Structure):
    """egpt_gemv_fused: one int8 GEMV of a single row with a fused prologue / epilogue."""
    _fields_ = [('epilogue', _c_int), ('N', _c_int), ('K', _c_int),
                ('x', _c_vp), ('x_token', _c_vp), ('x_ld', _c_i64), ('x_rows', _c_int),
                ('norm_w', _c_vp), ('eps', _c_f),
                ('merge_m', _c_vp), ('merge_l', _c_vp), ('merge_acc', _c_vp),
                ('merge_splits', _c_int), ('head_dim', _c_int),
                ('w', _c_vp), ('ldw', _c_i64), ('scale', _c_vp), ('y', _c_vp),
                ('resid', _c_vp), ('resid_token', _c_vp), ('resid_ld', _c_i64),
                ('part_v', _c_vp), ('part_i', _c_vp)]

    def weight_rows(self):
        """Rows of int8 weights the call streams (SwiGLU reads gate and up rows)."""
        return 2 * self.N if self.epilogue == EPI_SWIGLU else self.N

    def algorithmic_bytes(self):
        """Weights + scales + activation in + output out, the int8 GEMV byte model
        (N K + 4 N + 2 K + 2 N per output row set)."""
        rows = self.weight_rows()
        return rows * self.K + 4 * rows + 2 * self.K + 2 * self.N

_LAYER_FIELDS = ('qkv_w', 'qkv_s', 'o_w', 'o_s', 'gu_w', 'gu_s', 'down_w', 'down_s', 'in_norm', 'post_norm',
                 'q_norm', 'k_norm', 'k_cache', 'v_cache')


class Qwen3Layer(ctypes.Structure):
    """egpt_qwen3_layer: device pointers of one decoder layer."""
    _fields_ = [(name, _c_vp) for name in _LAYER_FIELDS]


class Qwen3Step(ctypes.Structure):
    """egpt_qwen3_step: shapes, weights, state and workspace of one fused decode step."""
    _fields_ = ([(name, _c_int) for name in ('layers', 'hidden', 'inter', 'heads', 'kv_heads', 'head_dim', 'vocab',
                                             'cap', 'nsplit')]
                + [('eps', _c_f)]
                + [(name, _c_vp) for name in ('layer', 'embed', 'final_norm', 'head_w', 'head_s', 'rope_cos',
                                              'rope_sin', 'token', 'position', 'x', 'qkv', 'attn', 'act', 'logits',
                                              'workspace')]
                + [('workspace_bytes', _c_size), ('token_ring', _c_vp), ('token_ring_slots', _c_int)])

_lib = None


class EgptError(RuntimeError):
    """A libegpt_hip entry point returned a non-zero status."""

    def __init__(self, name, status):
        self.status = status
        msg = lib().egpt_status_string(status).decode() if _lib is not None else str(status)
        super().__init__(f'{name} failed: {msg} ({status})')


def lib():
    """The loaded library, with argtypes set. Raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise ImportError(f'{LIB_PATH} is not built: run `python -m efficientgpt_amd._build` '
                              '(or __graft_entry__.build())')
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        got = handle.egpt_abi_version()
        if got != ABI_VERSION:
            raise ImportError(f'{LIB_PATH} has ABI {got}, expected {ABI_VERSION}: rebuild it')
        _lib = handle
    return _lib


def check(name, status):
    if status != EGPT_OK:
        raise EgptError(name, status)


_hip = None


def host_device_pointer(host_ptr):
    """The device address of pinned host memory (hipHostGetDevicePointer in the HIP runtime torch loaded), or None
    where the runtime does not map it."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL('libamdhip64.so.7', mode=ctypes.RTLD_GLOBAL)
        _hip.hipHostGetDevicePointer.restype = _c_int
        _hip.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(_c_vp), _c_vp, ctypes.c_uint]
    dev = _c_vp()
    if _hip.hipHostGetDevicePointer(ctypes.byref(dev), host_ptr, 0) != 0 or not dev.value:
        return None
    return dev.value


def stream_ptr(device=None):
    """The raw hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype):
    try:
        return {torch.float32: EGPT_F32, torch.bfloat16: EGPT_BF16, torch.float16: EGPT_F16}[dtype]
    except KeyError:
        raise ValueError(f'unsupported dtype {dtype}') from None
