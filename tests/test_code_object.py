"""The built library's gfx950 code objects: no kernel keeps any per-lane scratch memory.

A private segment means a local array the compiler could not keep in registers (a dynamically
indexed array, or an address taken through a pointer select). Each one has cost the decode step
dearly on the MI355X (a stack round trip on its critical path), so the build is checked for it.
Reads the code objects of libegpt_hip.so, built here; no GPU is used.
"""

import os
import re
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / 'efficientgpt_amd' / 'libegpt_hip.so'
LLVM = Path(os.environ.get('ROCM_PATH', '/opt/rocm')) / 'llvm' / 'bin'
TOOLS = [LLVM / 'llvm-objcopy', LLVM / 'clang-offload-bundler', LLVM / 'llvm-readelf']
MAGIC = b'__CLANG_OFFLOAD_BUNDLE__'


def kernel_metadata():
    """(kernel name, private segment bytes, vgpr spills) for every gfx950 kernel in the library."""
    out = []
    with tempfile.TemporaryDirectory() as tmp:
        fat = Path(tmp) / 'fatbin'
        subprocess.run([str(TOOLS[0]), f'--dump-section=.hip_fatbin={fat}', str(LIB), str(Path(tmp) / 'stripped')],
                       check=True, capture_output=True)
        data = fat.read_bytes()
        starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
        assert starts, 'no offload bundle in the library'
        for i, s in enumerate(starts):
            chunk = Path(tmp) / f'b{i}'
            chunk.write_bytes(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
            co = Path(tmp) / f'co{i}.o'
            subprocess.run([str(TOOLS[1]), '--unbundle', '--type=o', '--targets=hipv4-amdgcn-amd-amdhsa--gfx950',
                            f'--input={chunk}', f'--output={co}'], check=True, capture_output=True)
            notes = subprocess.run([str(TOOLS[2]), '--notes', str(co)], check=True, capture_output=True,
                                   text=True).stdout
            for blk in notes.split('  - .agpr_count:')[1:]:
                name = re.search(r'\.name:\s+(\S+)', blk).group(1)
                priv = int(re.search(r'\.private_segment_fixed_size:\s+(\d+)', blk).group(1))
                spill = int(re.search(r'\.vgpr_spill_count:\s+(\d+)', blk).group(1))
                out.append((name, priv, spill))
    return out


@pytest.mark.skipif(not LIB.is_file() or not all(t.is_file() for t in TOOLS), reason='library or ROCm tools missing')
def test_no_kernel_uses_scratch_memory():
    meta = kernel_metadata()
    names = [n for n, _, _ in meta]
    assert len(meta) > 50 and any('fused_gemv_kernel' in n for n in names) and any('attn_step_kernel' in n for n in names)
    bad = [(n, p, s) for n, p, s in meta if p or s]
    assert not bad, bad[:10]
