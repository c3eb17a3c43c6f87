"""bench.py's contract on the host: one GPU is measured, and any other count exits with a message.

Runs bench.py as the driver does (a child process); nothing here touches a GPU.
"""

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu_with_a_json_message():
    proc = subprocess.run([sys.executable, str(ROOT / 'bench.py'), '--gpus', '2', '--steps', '1', '--warmup', '0'],
                          capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert proc.returncode == 2, (proc.returncode, proc.stderr[-2000:])
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert line['n_gpus'] == 2 and 'one GPU' in line['error']


def test_bench_help_lists_the_contract_flags():
    proc = subprocess.run([sys.executable, str(ROOT / 'bench.py'), '--help'], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)
    assert proc.returncode == 0
    for flag in ('--gpus', '--steps', '--warmup'):
        assert flag in proc.stdout


def test_bench_cpu_name_reads_the_model():
    sys.path.insert(0, str(ROOT))
    import bench
    name = bench.cpu_name()
    assert isinstance(name, str) and name
    if Path('/proc/cpuinfo').exists() and 'model name' in Path('/proc/cpuinfo').read_text():
        assert name != 'x86_64'
