"""Batch-1 int8 decode benchmark on one MI355X.

Workload: a random-init Qwen3-1.7B-architecture model (28 layers, hidden 2048,
intermediate 6144, 16 q / 8 kv heads, head_dim 128, vocab 151936, tied
embeddings, RoPE theta 1e6), every linear int8 weight-only with per-output-channel
scales, weights N(0, 0.02); a 128-token uniform-random prompt is prefilled, then
each step is one replay of the captured decode graph (embedding through argmax and
the token / position update) producing one token. Weights, cache and prompt are
resident in HBM before timing starts.

Prints one JSON line:
  value        decode tokens/s over the timed steps (GPU-side, back-to-back replays)
  roofline     the int8 GEMV launches of one step (the dominant kernel), timed as a
               group with HIP events on their stream: algorithmic bytes / time vs the
               8 TB/s HBM peak
  cpu_baseline the CPU oracle (oracle/qwen3.py, torch on the host) on a bounded sample:
               prefill of the same prompt, then a few greedy decode steps
"""

import argparse
import json
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=256)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--model', choices=('qwen3-1.7b', 'qwen3-8b'), default='qwen3-1.7b')
    ap.add_argument('--prompt', type=int, default=128)
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--cpu-tokens', type=int, default=8, help='decode steps in the CPU baseline sample (0: skip)')
    ap.add_argument('--no-stream', action='store_true', help='skip the streamed generate() measurement')
    return ap.parse_args()


def gemv_roofline(eng, reps=20):
    """Time the int8 GEMV launches of one decode step (same shapes and buffers) as a captured graph."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    c = eng.cfg
    calls = []
    nbytes = 0

    def add(x, q, s, y):
        nonlocal nbytes
        n, k = q.shape
        nbytes += n * k + 4 * n + 2 * k + 2 * n
        calls.append((x, q, s, y))

    for L in eng.layers:
        add(eng.h, L['qkv_q'], L['qkv_s'], eng.qkv)
        add(eng.attn, L['o_q'], L['o_s'], eng.o)
        add(eng.h, L['gu_q'], L['gu_s'], eng.gu)
        add(eng.act, L['down_q'], L['down_s'], eng.down)
    add(eng.h, eng.head_q, eng.head_s, eng.logits)

    def run():
        st = _lib.stream_ptr(eng.device)
        for x, q, s, y in calls:
            _lib.check('egpt_int8_gemv', lib.egpt_int8_gemv(x.data_ptr(), x.stride(0), q.data_ptr(), q.stride(0),
                                                            s.data_ptr(), y.data_ptr(), y.stride(0), 1, q.shape[0],
                                                            q.shape[1], st))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    per_step_s = e0.elapsed_time(e1) / 1e3 / reps
    launches = len(calls)
    achieved = nbytes / per_step_s / 1e9
    return {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
            'frac': round(achieved / HBM_PEAK_GBPS, 4), 'traffic': None,
            'kernel': 'egpt int8 GEMV (gemv_i8_rows), all launches of one decode step',
            'launches': launches, 'bytes_per_step': nbytes,
            'avg_launch_us': round(per_step_s / launches * 1e6, 3),
            'gemv_ms_per_step': round(per_step_s * 1e3, 4)}


def host_threads():
    """CPU threads this process may use: OMP_NUM_THREADS if set, else the cores in its affinity mask."""
    env = os.environ.get('OMP_NUM_THREADS')
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0)) or 1


def cpu_baseline(eng, prompt, n_tokens, gpu_tokens):
    """The CPU oracle on the same weights: prefill the prompt, then n_tokens greedy steps."""
    from oracle.qwen3 import Qwen3Oracle, Qwen3Shape
    c = eng.cfg
    torch.set_num_threads(host_threads())
    shape = Qwen3Shape(c.vocab, c.hidden, c.inter, c.layers, c.heads, c.kv_heads, c.head_dim, c.rope_theta,
                       c.rms_eps, c.tied)
    w = {k: v.cpu() for k, v in eng.weights.items()}
    orc = Qwen3Oracle(shape, w, dtype=torch.bfloat16, cap=len(prompt) + n_tokens + 1)
    t0 = time.perf_counter()
    logits = orc.forward(prompt, 0)
    toks = [int(torch.argmax(logits))]
    t_first = time.perf_counter()
    pos = len(prompt)
    for _ in range(n_tokens - 1):
        logits = orc.forward([toks[-1]], pos)
        pos += 1
        toks.append(int(torch.argmax(logits)))
    t1 = time.perf_counter()
    decode_tps = (n_tokens - 1) / (t1 - t_first) if n_tokens > 1 else None
    agree = sum(a == b for a, b in zip(toks, gpu_tokens[:n_tokens]))
    return {'value': round(decode_tps, 3) if decode_tps else None, 'unit': 'tok/s', 'cores': torch.get_num_threads(),
            'kind': 'port',
            'sample': (f'CPU oracle (torch, bf16 activations, fp32 image of the int8 weights) on the same weights: '
                       f'prefill of the {len(prompt)}-token prompt ({t_first - t0:.1f} s) then {n_tokens} greedy '
                       f'tokens; decode tok/s = (n-1)/(decode time)'),
            'cpu': platform.processor() or platform.machine(),
            'token_agreement_with_gpu': f'{agree}/{n_tokens}'}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({'error': 'this build runs on one GPU; multi-GPU runs are not part of it',
                          'n_gpus': args.gpus}))
        sys.exit(2)
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    from efficientgpt_amd.qwen3 import QWEN3_1_7B, QWEN3_8B, Qwen3Int8Engine

    cfg = QWEN3_1_7B if args.model == 'qwen3-1.7b' else QWEN3_8B
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    n_stream = 256
    cap = args.prompt + max(args.warmup + args.steps, n_stream) + 8
    t = time.perf_counter()
    eng = Qwen3Int8Engine.random(cfg, cap, seed=args.seed, device=dev)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t
    prompt = torch.randint(0, cfg.vocab, (args.prompt,), generator=torch.Generator().manual_seed(args.seed + 1))

    with torch.inference_mode():
        # GPU decode: prefill, capture, warm-up replays, then K timed replays back to back
        eng.reset()
        eng.prefill(prompt)
        eng.capture()
        tokens = [int(eng.token)]
        for _ in range(args.warmup):
            eng.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            eng.graph.replay()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gpu_s = e0.elapsed_time(e1) / 1e3
        value = args.steps / wall

        roof = gemv_roofline(eng)

        stream = None
        gpu_tokens = []
        if not args.no_stream:
            dec = GraphGreedyDecoder(eng, max_cache_len=cap)
            out, st = dec.generate(prompt.view(1, -1).to(dev), n_stream)
            gpu_tokens = out
            stream = {'decode_tok_s': round((st['tokens'] - 1) / (st['total_s'] - st['ttft_s']), 2),
                      'ttft_ms': round(st['ttft_s'] * 1e3, 2), 'tokens': st['tokens'],
                      'distinct_tokens': len(set(out))}
    cpu = cpu_baseline(eng, prompt, args.cpu_tokens, gpu_tokens) if args.cpu_tokens > 0 and gpu_tokens else None

    wbytes, sbytes = cfg.weight_bytes()
    line = {
        'metric': 'batch-1 decode tok/s (Qwen3-1.7B-shape int8); GEMV/attn HBM GB/s vs peak',
        'value': round(value, 2), 'unit': 'tok/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': round(wall / args.steps * 1e3, 4), 'gpu_ms_per_step': round(gpu_s / args.steps * 1e3, 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'int8 weights, bf16 activations, fp32 accumulation',
        'data': 'synthetic: random-init weights N(0,0.02), uniform-random prompt ids',
        'config': {'workload': f'{args.model} int8 batch-1 greedy decode, {args.prompt}-token prompt, one graph replay per token',
                   'model': args.model, 'global_batch': 1, 'seq_len': args.prompt + args.warmup + args.steps,
                   'parallelism': 'single GPU'},
        'roofline': roof,
        'cpu_baseline': cpu,
        'streamed_generate': stream,
        'step_bytes': {'int8_weights': wbytes, 'scales': sbytes, 'kv_per_slot': cfg.kv_bytes_per_slot()},
        'build_s': round(build_s, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
