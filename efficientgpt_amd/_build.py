"""Builds libegpt_hip.so in-tree from the HIP sources in csrc/ (gfx950 only).

`python -m efficientgpt_amd._build` compiles every time it is called. The library
is written next to this file so it travels with the source tree.
"""

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / 'csrc'
LIB = PKG / 'libegpt_hip.so'
ARCH = 'gfx950'

HIPCC_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared',
    # hipcc -O3 forms packed-fp32 instructions from float code on its own; some of
    # their forms have given silently wrong results on the target machines, so
    # they are switched off for every kernel. The host pass warns that it does not
    # know the feature; that is expected.
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wno-unused-command-line-argument',
    f'-I{ROOT / "include"}',
]


def sources():
    return sorted(str(p) for p in CSRC.glob('*.hip'))


def hipcc():
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    path = Path(rocm) / 'bin' / 'hipcc'
    return str(path) if path.exists() else 'hipcc'


def build(verbose=False):
    """Compile csrc/*.hip into libegpt_hip.so (atomic replace). Raises on failure."""
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [hipcc(), *HIPCC_FLAGS, *sources(), '-o', str(tmp)]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}')
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
