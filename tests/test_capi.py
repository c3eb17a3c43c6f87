"""The C ABI library loads and exports exactly what include/egpt.h declares (CPU: no kernel launches)."""

import ctypes
import re
from pathlib import Path

import pytest

from efficientgpt_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / 'include' / 'egpt.h'


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(egpt_[a-z0-9_]+)\s*\(', text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.egpt_abi_version() == _lib.ABI_VERSION
    assert lib.egpt_status_string(0) == b'ok'


def test_argument_errors_return_status_without_launching():
    lib = _lib.lib()
    dummy = ctypes.c_void_p(16)
    # null operands
    assert lib.egpt_int8_gemv(None, 0, dummy, 16, dummy, dummy, 0, 1, 16, 16, None) == -1
    # more rows than the decode kernel takes
    assert lib.egpt_int8_gemv(dummy, 16, dummy, 16, dummy, dummy, 16, 17, 16, 16, None) == -2
    # row stride shorter than K
    assert lib.egpt_int8_gemv(dummy, 16, dummy, 8, dummy, dummy, 16, 1, 16, 16, None) == -1
    size = ctypes.c_size_t()
    assert lib.egpt_int8_gemv_splitk_workspace(2, 100, 64, 4, ctypes.byref(size)) == 0
    assert size.value == 4 * 2 * 100 * 4
    assert lib.egpt_int8_gemv_splitk(dummy, 64, dummy, 64, dummy, dummy, 100, 2, 100, 64, 4, None, 0, None) == -4
    # attention: Hq not a multiple of Hkv, unsupported dtype, missing workspace
    args = [dummy, 0, 0, dummy, 0, 0, 0, dummy, 0, 0, 0, dummy, 0, dummy, 0, 0]
    assert lib.egpt_decode_attn(1, *args, None, 0, 1, 6, 4, 64, 128, 1, 0.1, None) == -1
    assert lib.egpt_decode_attn(7, *args, None, 0, 1, 8, 4, 64, 128, 1, 0.1, None) == -2
    assert lib.egpt_decode_attn(1, *args, None, 0, 1, 8, 4, 64, 128, 1, 0.1, None) == -4
    assert lib.egpt_decode_attn_workspace(1, 16, 8, 4096, 128, 8, ctypes.byref(size)) == 0
    assert size.value >= 16 * 8 * (128 + 2) * 4
    # the allocation-free form: more partials than its scratch array holds (16 heads x 505 splits at D 128)
    assert lib.egpt_decode_attn_workspace(1, 16, 8, 4096, 128, 505, ctypes.byref(size)) == 0
    assert size.value > _lib.NOALLOC_SCRATCH_BYTES
    assert lib.egpt_decode_attn_noalloc(1, *args, 1, 16, 8, 4096, 128, 505, 0.1, None) == -4
    assert lib.egpt_decode_attn_noalloc(1, *args, 0, 16, 8, 4096, 128, 1, 0.1, None) == -1
    # quantisation: null codes, row stride shorter than K, unknown dtype; no rows is a no-op
    assert lib.egpt_quantize_rows(0, dummy, 64, 4, 64, None, 64, dummy, None) == -1
    assert lib.egpt_quantize_rows(0, dummy, 32, 4, 64, dummy, 64, dummy, None) == -1
    assert lib.egpt_quantize_rows(9, dummy, 64, 4, 64, dummy, 64, dummy, None) == -2
    assert lib.egpt_quantize_rows(1, dummy, 64, 0, 64, dummy, 64, dummy, None) == 0


@pytest.mark.parametrize('b,hkv,cap', [(1, 8, 256), (1, 8, 32768), (16, 6, 128), (1, 1, 1)])
def test_default_splits_bounded(b, hkv, cap):
    n = _lib.lib().egpt_decode_attn_default_splits(b, hkv, cap)
    assert 1 <= n <= 256 and n <= max(1, cap)


def test_split_policies():
    """The stand-alone attention runs one pass up to 256 slots and wherever 256 (row, kv head) programs fill the
    GPU; past that about one block per CU with at least 64 slots per split. The decode step splits short caches
    too (its merge needs no launch of its own). Host functions: no GPU is touched."""
    from efficientgpt_amd.decode_attention import use_single_pass
    lib = _lib.lib()
    for b, hkv in ((1, 8), (4, 6), (16, 8), (32, 8), (64, 6)):
        for cap in (1, 2, 63, 64, 65, 128, 255, 256, 257, 400, 1024, 4096, 32768, 131072):
            n = lib.egpt_decode_attn_default_splits(b, hkv, cap)
            assert (n == 1) == use_single_pass(b, hkv, cap), (b, hkv, cap, n)
            if cap > 256:
                assert n == min(-(-cap // 64), -(-256 // (b * hkv)), 256), (b, hkv, cap, n)
    step = lib.egpt_qwen3_step_default_splits
    # Qwen3-1.7B geometry (16 / 8 heads, D 128): up to 3072 slots (attention blocks of one query head) at most 4
    # splits to 512 slots and 8 past that; then about one block per CU
    assert [step(16, 8, 128, c) for c in (64, 96, 256, 400, 512, 513, 1024, 1772, 2048, 3072, 3073, 32768)] == \
        [1, 2, 4, 4, 4, 8, 8, 8, 8, 8, 32, 32]
    # Qwen3-8B geometry (32 / 8 heads)
    assert [step(32, 8, 128, c) for c in (400, 964, 1772, 2048, 2112, 3072, 3136, 8192)] == [4, 8, 8, 8, 8, 8, 32, 32]
    assert step(4, 2, 32, 4096) == 64
    assert step(0, 8, 128, 100) == 1 and step(16, 0, 128, 100) == 1


def test_struct_layouts_match_the_header(tmp_path):
    """The ctypes mirrors of egpt_gemv_fused / egpt_qwen3_step / egpt_qwen3_layer have the C layout."""
    import shutil
    import subprocess
    gcc = shutil.which('gcc')
    if gcc is None:
        pytest.skip('gcc not available')
    src = tmp_path / 'layout.c'
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "egpt.h"\n'
                   'int main(void) {\n'
                   '  printf("%zu %zu %zu %zu %zu %zu %zu\\n", sizeof(egpt_gemv_fused), offsetof(egpt_gemv_fused, part_i),\n'
                   '         offsetof(egpt_gemv_fused, w), sizeof(egpt_qwen3_step),\n'
                   '         offsetof(egpt_qwen3_step, workspace_bytes), sizeof(egpt_qwen3_layer),\n'
                   '         offsetof(egpt_qwen3_step, token_ring_slots));\n'
                   '  return 0;\n}\n')
    exe = tmp_path / 'layout'
    subprocess.run([gcc, '-D__HIP_PLATFORM_AMD__', f'-I{HEADER.parent}', '-I/opt/rocm/include', str(src), '-o', str(exe)],
                   check=True, capture_output=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    want = [ctypes.sizeof(_lib.GemvFused), _lib.GemvFused.part_i.offset, _lib.GemvFused.w.offset,
            ctypes.sizeof(_lib.Qwen3Step), _lib.Qwen3Step.workspace_bytes.offset, ctypes.sizeof(_lib.Qwen3Layer),
            _lib.Qwen3Step.token_ring_slots.offset]
    assert got == want


def test_gemm_split_workspace_policy():
    """Short-M prefill shapes split K until every CU has a block (at most 16 splits, at least 4 K steps of 64
    each); past 128 rows (up to 256) only grids of at most 128 tiles split; tall ones and short K do not split."""
    lib = _lib.lib()
    size = ctypes.c_size_t()
    for (m, n, k), splits in (((128, 2048, 6144), 4), ((128, 4096, 2048), 2), ((64, 2048, 2048), 8),
                              ((17, 64, 12288), 16), ((128, 12288, 2048), 0), ((1024, 2048, 6144), 0),
                              ((128, 2048, 256), 0), ((200, 2048, 2048), 2), ((130, 2048, 2048), 4),
                              ((160, 4096, 2048), 0), ((256, 2048, 6144), 2), ((257, 2048, 2048), 0)):
        assert lib.egpt_int8_gemm_workspace(m, n, k, ctypes.byref(size)) == 0
        assert size.value == splits * m * n * 4, (m, n, k, size.value)
