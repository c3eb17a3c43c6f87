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
    # Leading scalar and pointer kernel arguments are preloaded into registers at
    # launch (gfx950 kernel-argument preload), so a kernel's first loads need no
    # read of its argument block; structs passed by value are not preloaded.
    '-mllvm', '-amdgpu-kernarg-preload-count=16',
    '-Wno-unused-command-line-argument',
    f'-I{ROOT / "include"}',
]


def sources():
    return sorted(str(p) for p in CSRC.glob('*.hip'))


def hipcc():
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    path = Path(rocm) / 'bin' / 'hipcc'
    return str(path) if path.exists() else 'hipcc'


def _run(cmd, verbose):
    if verbose:
        print(' '.join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def build(verbose=False, jobs=None):
    """Compile csrc/*.hip into libegpt_hip.so (atomic replace). Raises on failure.

    Each source is compiled to its own object in parallel (the translation units share
    no device symbols), then the objects are linked into the shared library."""
    objdir = PKG / '_build'
    objdir.mkdir(exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 1)
    compile_flags = [f for f in HIPCC_FLAGS if f != '-shared']
    pending = [(src, objdir / (Path(src).stem + '.o')) for src in sources()]
    running, objects = [], []
    while pending or running:
        while pending and len(running) < jobs:
            src, obj = pending.pop(0)
            objects.append(obj)
            running.append((src, _run([hipcc(), *compile_flags, '-c', src, '-o', str(obj)], verbose)))
        src, proc = running.pop(0)
        _, err = proc.communicate()
        if proc.returncode != 0:
            for _, other in running:
                other.kill()
            raise RuntimeError(f'hipcc failed on {src} ({proc.returncode}):\n{err[-4000:]}')
    tmp = LIB.with_suffix('.so.tmp')
    link = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, objects), '-o', str(tmp)]
    proc = _run(link, verbose)
    _, err = proc.communicate()
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc link failed ({proc.returncode}):\n{err[-4000:]}')
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
