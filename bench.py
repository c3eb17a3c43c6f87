"""Batch-1 int8 decode benchmark on one MI355X.

Workload (default): a random-init Qwen3-1.7B-architecture model (28 layers,
hidden 2048, intermediate 6144, 16 q / 8 kv heads, head_dim 128, vocab 151936,
tied embeddings, RoPE theta 1e6), every linear int8 weight-only with
per-output-channel scales, weights N(0, 0.02); a 128-token uniform-random prompt
is prefilled, then each step is one replay of the captured decode graph
(embedding through argmax and the token / position update) producing one token.
`--model qwen3-8b --prompt 8192` runs the long-context 8B workload instead.
Weights, cache and prompt are resident in HBM before timing starts.

Prints one JSON line:
  value           decode tokens/s over K back-to-back graph replays: the median of --rounds
                  rounds (5), each from the state the prefill left; `spread` holds every
                  round, the min and max, and the GPU's busy percentage read when the process
                  starts, before it has run anything on the GPU (`contended` when above 10%:
                  other work on the card); `host_cpu` the CPU model from /proc/cpuinfo
  roofline        the dominant kernel, the fused int8 GEMV (fused_gemv_kernel): the
                  step's own GEMV launches (egpt_qwen3_step_gemvs, 4 per layer + the
                  lm_head) replayed as one graph through egpt_int8_gemv_fused and timed
                  with HIP events on their stream; algorithmic bytes (int8 weights +
                  fp32 scales + bf16 activation in / out) over the average launch time.
                  The set streams > 1.7 GB per pass, so it is HBM-cold by construction.
  attention       split-K decode attention at the largest context of the workload
                  family (16 q / 8 kv heads, D 128, L = 32768), rotating > 512 MB of K/V
  attention_by_length  the same at L = 256 ... 16384
  gemv_1x2048_6144     the reference's headline GEMV shape through egpt_int8_gemv, cold
  prefill_gemm         the MFMA prefill GEMM at the model's shapes, beside the reference's formula
  launch_floor_us the fixed cost of one dependent GEMV launch in a graph (a one-row GEMV
                  whose 2 KB of weights come from HBM); `frac_beyond_floor` beside a small
                  kernel's `frac` takes one floor per launch out of its time
  gemv_small_batch     egpt_int8_gemv at each Qwen3-1.7B GEMV shape and the lm_head with
                  1, 2, 4 and 8 activation rows, cold
  long_context    the Qwen3-8B workload: 8192-token prompt, cache of 8704 slots, graph
                  replays timed, its GEMV launches timed on their own
  step            the whole step: weight + scale + KV bytes per token / ms per token
  copy_gbps       a device-to-device copy of 1 GiB, the measured bandwidth ceiling
  cpu_baseline    the CPU oracle (oracle/qwen3.py, torch on the host) on the same
                  workload: prefill of the same prompt, then all 256 greedy tokens
                  (--cpu-tokens sets fewer), on the same weights; `kernels` holds the reference's CPU forms of the GEMV (every
                  shape, 1-8 rows) and the attention (every cache length) timed on the host
"""

import argparse
import ctypes
import itertools
import json
import math
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=256)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--model', choices=('qwen3-1.7b', 'qwen3-8b'), default='qwen3-1.7b')
    ap.add_argument('--prompt', type=int, default=128)
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--rounds', type=int, default=5,
                    help='timed rounds of the same K steps; value is the median round (min and max reported)')
    ap.add_argument('--cpu-tokens', type=int, default=256,
                    help='greedy tokens of the CPU baseline (0: skip; the default 256 is the whole decode of the workload)')
    ap.add_argument('--cpu-long-tokens', type=int, default=4,
                    help='CPU decode steps timed on the Qwen3-8B long-context weights (0: skip)')
    ap.add_argument('--no-long-context', action='store_true',
                    help='skip the Qwen3-8B long-context measurement (8192-token prompt)')
    ap.add_argument('--no-stream', action='store_true', help='skip the streamed generate() measurement')
    ap.add_argument('--no-extra', action='store_true', help='skip the attention and copy measurements')
    ap.add_argument('--attention-only', default=None, metavar='L[,L...]',
                    help='instead of the decode benchmark: the stand-alone split-K attention at these cache lengths '
                         '(one JSON line each, cold), with --heads query / kv heads at head_dim 128')
    ap.add_argument('--heads', default='16/8', help='query / kv heads for --attention-only (default 16/8)')
    ap.add_argument('--dispatch-grid', action='store_true',
                    help='instead of the decode benchmark: single-pass against default split-K decode attention over '
                         'batch x heads x cache length (one JSON line per point), the data behind the split policy')
    return ap.parse_args()


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _time_graph(fn, reps):
    """Capture fn() (launches on the current stream) as one graph; mean seconds per replay."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = _events()
    e0.record()  # on the current stream, the one the graph replays on
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def gemv_roofline(eng, reps=20):
    """The step's fused GEMV launches, replayed through the public entry point, as one graph."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    n = ctypes.c_int()
    _lib.check('egpt_qwen3_step_gemvs', lib.egpt_qwen3_step_gemvs(ctypes.byref(eng._step_c), None, 0, ctypes.byref(n)))
    descs = (_lib.GemvFused * n.value)()
    _lib.check('egpt_qwen3_step_gemvs', lib.egpt_qwen3_step_gemvs(ctypes.byref(eng._step_c), descs, n.value,
                                                                  ctypes.byref(n)))
    nbytes = sum(d.algorithmic_bytes() for d in descs)
    head = descs[n.value - 1]

    def run():
        st = _lib.stream_ptr()
        for d in descs:
            _lib.check('egpt_int8_gemv_fused', lib.egpt_int8_gemv_fused(ctypes.byref(d), st))

    per_pass = _time_graph(run, reps)
    achieved = nbytes / per_pass / 1e9
    return {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
            'frac': round(achieved / HBM_PEAK_GBPS, 4), 'traffic': None,
            'kernel': 'fused_gemv_kernel (int8 GEMV, RMSNorm / residual / SwiGLU / argmax fused), '
                      'the decode step\'s own launches',
            'launches': n.value, 'bytes_per_launch': round(nbytes / n.value),
            'bytes_per_step': nbytes, 'avg_launch_us': round(per_pass / n.value * 1e6, 3),
            'gemv_ms_per_step': round(per_pass * 1e3, 4),
            'units': f'{4 * eng.cfg.layers} layer GEMVs (QKV {head.K}x{(eng.cfg.heads + 2 * eng.cfg.kv_heads) * eng.cfg.head_dim}, '
                     f'o_proj, gate/up, down) + lm_head {head.N}x{head.K}'}


TRAFFIC_SUMMARY = os.path.join(ROOT, 'profiles', 'fused_gemv_traffic_qwen3_1p7b.md')


def measured_traffic(model):
    """HBM bytes per fused-GEMV launch of the Qwen3-1.7B step, from the two calibrated rocprofv3 --pmc runs
    (FETCH_SIZE, WRITE_SIZE) summarised in profiles/; None for other workloads or without the summary."""
    if model != 'qwen3-1.7b' or not os.path.isfile(TRAFFIC_SUMMARY):
        return None
    with open(TRAFFIC_SUMMARY) as f:
        for line in f:
            if line.startswith('traffic_bytes_per_launch:'):
                return int(line.split(':', 1)[1])
    return None


def attention_roofline(L=32768, hq=16, hkv=8, d=128, copies=4, reps=5):
    """Split-K GQA decode attention over all L slots, rotating `copies` K/V sets (> 512 MB)."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    dev = torch.device('cuda')
    g = torch.Generator(device=dev).manual_seed(7)
    ks = [torch.randn(1, hkv, L, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    vs = [torch.randn(1, hkv, L, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    q = torch.randn(1, hq, 1, d, generator=g, device=dev).to(torch.bfloat16)
    pos = torch.tensor([L - 1], device=dev)
    out = torch.empty_like(q)
    nsplit = lib.egpt_decode_attn_default_splits(1, hkv, L)
    need = ctypes.c_size_t()
    _lib.check('ws', lib.egpt_decode_attn_workspace(1, hq, hkv, L, d, nsplit, ctypes.byref(need)))
    ws = torch.empty(need.value, device=dev, dtype=torch.uint8)

    def run():
        st = _lib.stream_ptr()
        for k, v in zip(ks, vs):
            _lib.check('egpt_decode_attn', lib.egpt_decode_attn(
                _lib.EGPT_BF16, q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), pos.data_ptr(), 0, out.data_ptr(),
                out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(), 1, hq, hkv, L, d, nsplit, d ** -0.5, st))

    per_call = _time_graph(run, reps) / copies
    nbytes = 2 * hkv * L * d * 2 + 2 * (2 * hq * d)
    achieved = nbytes / per_call / 1e9
    del ks, vs
    torch.cuda.empty_cache()
    return {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
            'frac': round(achieved / HBM_PEAK_GBPS, 4), 'L': L, 'nsplit': nsplit,
            'bytes_per_call': nbytes, 'us_per_call': round(per_call * 1e6, 2),
            'kernel': 'attn_split_kernel + attn_combine_kernel (egpt_decode_attn), cold'}


def gemv_cfg0(n=6144, k=2048, sets=48, reps=10):
    """The reference's headline GEMV, one 2048-wide row times 6144 x 2048 int8 weights
    (research/kernelagent/tasks.py:206-209), through egpt_int8_gemv over `sets` rotating weight
    copies (> 512 MB) captured in one graph, so every call streams its weights from HBM."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    dev = torch.device('cuda')
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16)
    ws = [torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8) for _ in range(sets)]
    sc = torch.randn(n, generator=g, device=dev).abs() * 0.02 / 127
    y = torch.empty(1, n, device=dev, dtype=torch.bfloat16)

    def run():
        st = _lib.stream_ptr()
        for w in ws:
            _lib.check('egpt_int8_gemv', lib.egpt_int8_gemv(x.data_ptr(), k, w.data_ptr(), k, sc.data_ptr(),
                                                            y.data_ptr(), n, 1, n, k, st))

    per_call = _time_graph(run, reps) / sets
    nbytes = n * k + 4 * n + 2 * k + 2 * n
    del ws
    torch.cuda.empty_cache()
    return {'bound': 'hbm', 'achieved': round(nbytes / per_call / 1e9, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
            'frac': round(nbytes / per_call / 1e9 / HBM_PEAK_GBPS, 4), 'shape': f'1x{k} -> {n}',
            'bytes_per_call': nbytes, 'us_per_call': round(per_call * 1e6, 3),
            'kernel': 'egpt_int8_gemv (one aligned row: the fused kernel'"'"'s store variant), cold, one call per '
                      'weight copy, each call including its hand-off from the previous launch'}


def prefill_gemm(rows=(128, 1024), shapes=((4096, 2048), (12288, 2048), (2048, 6144), (2048, 2048)), reps=3):
    """The prefill GEMM (egpt_int8_gemm_ws, bf16 MFMA on int8 weights, K split over a workspace where the output
    tiles alone leave CUs idle) at Qwen3-1.7B's QKV, gate/up, down and o_proj shapes, beside the reference's formula for the same product (research/realmodel/int8_linear.py:96-97:
    dequantise to bf16, library GEMM, scale). TF/s of 2 M N K flops; peak dense bf16 MFMA 2500 TF/s."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    dev = torch.device('cuda')
    out = []
    for m in rows:
        for n, k in shapes:
            g = torch.Generator(device=dev).manual_seed(0)
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            q = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
            sc = torch.rand(n, generator=g, device=dev) * 1e-3
            y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
            calls = max(1, int(2e11 // (2 * m * n * k)))
            need = ctypes.c_size_t()
            _lib.check('egpt_int8_gemm_workspace', lib.egpt_int8_gemm_workspace(m, n, k, ctypes.byref(need)))
            ws = torch.empty(max(need.value, 16), device=dev, dtype=torch.uint8)

            def ours():
                for _ in range(calls):
                    _lib.check('egpt_int8_gemm_ws', lib.egpt_int8_gemm_ws(
                        x.data_ptr(), k, q.data_ptr(), k, sc.data_ptr(), y.data_ptr(), n, m, n, k, ws.data_ptr(),
                        need.value, _lib.stream_ptr()))

            def reference():
                for _ in range(calls):
                    ((x @ q.to(torch.bfloat16).t()).float() * sc).to(torch.bfloat16)

            t_ours = _time_graph(ours, reps) / calls
            t_ref = _time_graph(reference, reps) / calls
            fl = 2 * m * n * k
            out.append({'shape': f'{m}x{k} -> {n}', 'us': round(t_ours * 1e6, 1), 'k_splits': need.value // (m * n * 4),
                        'tflops': round(fl / t_ours / 1e12, 1), 'frac': round(fl / t_ours / 2.5e15, 4),
                        'reference_formula_us': round(t_ref * 1e6, 1)})
            del x, q, y
    torch.cuda.empty_cache()
    return out


def attention_sweep(lengths=(256, 1024, 4096, 16384)):
    """attention_roofline at shorter live lengths, each over > 512 MB of rotating K/V copies."""
    out = {}
    for L in lengths:
        r = attention_roofline(L=L, copies=max(4, (1 << 29) // (4096 * L) + 1), reps=3)
        out[str(L)] = {k: r[k] for k in ('achieved', 'frac', 'nsplit', 'us_per_call')}
    return out


def launch_floor(chain=64, reps=20):
    """The fixed cost of one dependent GEMV launch in a graph: `chain` egpt_int8_gemv calls of ONE 2048-wide output
    row each (2 KB of weights, 16 MB apart in a 1 GiB buffer, so every call's row comes from HBM), each reading the
    previous call's output. What a call costs beyond its own bytes: the launch boundary, the round trip of its first
    loads, its reduction and store. Each call is one block: with kernel arguments preloaded into registers a one-block
    launch costs about 0.12 us more, while launches of two blocks and more (every launch of the decode step) cost
    0.03-0.05 us less, so this floor reads about 0.1 us above theirs."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    dev = torch.device('cuda')
    k = 2048
    w = torch.randint(-127, 128, (1 << 30,), dtype=torch.int8, device=dev)
    sc = torch.full((1,), 1e-3, device=dev)
    xs = torch.randn(chain + 1, k, device=dev).to(torch.bfloat16)
    stride = (1 << 30) // chain

    def run():
        st = _lib.stream_ptr()
        for i in range(chain):
            # the output row is element 0 of the next call's activation row
            _lib.check('egpt_int8_gemv', lib.egpt_int8_gemv(xs[i].data_ptr(), k, w[i * stride:].data_ptr(), k,
                                                            sc.data_ptr(), xs[i + 1].data_ptr(), 1, 1, 1, k, st))

    us = _time_graph(run, reps) / chain * 1e6
    del w
    torch.cuda.empty_cache()
    return round(us, 3)


CONFIG1_SHAPES = (('qkv', 4096, 2048), ('o_proj', 2048, 2048), ('gate_up', 12288, 2048), ('down', 2048, 6144),
                  ('lm_head', 151936, 2048))


def gemv_small_batch(floor_us, rows=(1, 2, 4, 8), reps=5):
    """egpt_int8_gemv at each per-layer GEMV shape of Qwen3-1.7B and the lm_head, with M = 1, 2, 4, 8 activation
    rows, cold (each call streams its own weight copy; the copies of one shape total > 512 MB). Bytes per call are
    N K + 4 N + 2 M K + 2 M N; `frac_beyond_floor` takes the launch floor out of the time."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    dev = torch.device('cuda')
    out = {}
    for name, n, k in CONFIG1_SHAPES:
        sets = max(2, -(-(600 << 20) // (n * k)))
        g = torch.Generator(device=dev).manual_seed(1)
        ws = [torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8) for _ in range(sets)]
        sc = torch.rand(n, generator=g, device=dev) * 1e-3
        for m in rows:
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

            def run():
                st = _lib.stream_ptr()
                for w in ws:
                    _lib.check('egpt_int8_gemv', lib.egpt_int8_gemv(x.data_ptr(), k, w.data_ptr(), k, sc.data_ptr(),
                                                                    y.data_ptr(), n, m, n, k, st))

            t = _time_graph(run, reps) / sets
            nbytes = n * k + 4 * n + 2 * m * k + 2 * m * n
            gbps = nbytes / t / 1e9
            beyond = nbytes / max(t - floor_us * 1e-6, 1e-9) / 1e9
            out[f'{m}x{k}->{n}'] = {'shape': name, 'rows': m, 'us': round(t * 1e6, 2), 'achieved': round(gbps, 1),
                                   'frac': round(gbps / HBM_PEAK_GBPS, 4),
                                   'frac_beyond_floor': round(beyond / HBM_PEAK_GBPS, 4)}
        del ws
        torch.cuda.empty_cache()
    return out


# The reference's held-out small GEMV shapes (M x K -> N) and its published times on an RTX 4060, L2-warm
# (runs/20261031_v4/int8_study/heldout_int8_gemv.json; the reference does not claim them as DRAM numbers).
REFERENCE_HELDOUT_US = {(1, 2048, 2048): 7.6, (2, 2048, 1024): 5.3, (4, 6144, 2048): 20.1, (8, 2048, 6144): 22.2}


def gemv_reference_shapes(reps=5):
    """egpt_int8_gemv at the reference's held-out small shapes, warm (one weight copy, called back to back, so it
    stays in the caches as the reference's numbers do) and cold (a weight copy per call), beside the reference's
    published time."""
    from efficientgpt_amd import _lib
    lib = _lib.lib()
    dev = torch.device('cuda')
    g = torch.Generator(device=dev).manual_seed(2)
    out = {}
    for (m, k, n), ref_us in REFERENCE_HELDOUT_US.items():
        sets = max(2, -(-(600 << 20) // (n * k)))
        ws = [torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8) for _ in range(sets)]
        sc = torch.rand(n, generator=g, device=dev) * 1e-3
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

        def run(weights):
            st = _lib.stream_ptr()
            for w in weights:
                _lib.check('egpt_int8_gemv', lib.egpt_int8_gemv(x.data_ptr(), k, w.data_ptr(), k, sc.data_ptr(),
                                                                y.data_ptr(), n, m, n, k, st))

        cold = _time_graph(lambda: run(ws), reps) / sets
        warm = _time_graph(lambda: run([ws[0]] * sets), reps) / sets
        out[f'{m}x{k}->{n}'] = {'us_warm': round(warm * 1e6, 2), 'us_cold': round(cold * 1e6, 2),
                               'reference_rtx4060_warm_us': ref_us}
        del ws
        torch.cuda.empty_cache()
    return out


def cpu_long_context(cfg, weights, prompt_len, n_tokens, threads, seed=5):
    """The CPU oracle on the long-context model's weights, a stated subset of its decode: the 8192-token prefill
    is not run on the CPU (about 1.3e14 flops); the oracle's cache slots 0..prompt_len-1 are filled with seeded
    N(0, 1) bf16 keys and values instead, which costs a decode step exactly what the prefilled cache would, and
    n_tokens greedy steps are timed from position prompt_len. Decode tok/s = n_tokens / time (no TTFT in it)."""
    from oracle.qwen3 import Qwen3Oracle, Qwen3Shape
    torch.set_num_threads(threads)
    shape = Qwen3Shape(cfg.vocab, cfg.hidden, cfg.inter, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim,
                       cfg.rope_theta, cfg.rms_eps, cfg.tied)
    orc = Qwen3Oracle(shape, weights, dtype=torch.bfloat16, cap=prompt_len + n_tokens + 1)
    t = time.perf_counter()
    orc.forward([0], 0)  # builds the cached fp32 images of the int8 weights outside the timed run
    build_s = time.perf_counter() - t
    orc.reset()
    g = torch.Generator().manual_seed(seed)
    for layer in range(cfg.layers):
        for cache in (orc.k_cache[layer], orc.v_cache[layer]):
            cache[:, :prompt_len] = torch.randn(cfg.kv_heads, prompt_len, cfg.head_dim, generator=g).to(cache.dtype)
    tok, pos = 1, prompt_len
    t0 = time.perf_counter()
    for _ in range(n_tokens):
        tok = int(torch.argmax(orc.forward([tok], pos)))
        pos += 1
    dt = time.perf_counter() - t0
    del orc
    return {'value': round(n_tokens / dt, 3), 'unit': 'tok/s', 'cores': torch.get_num_threads(), 'kind': 'port',
            'sample': (f'CPU oracle on the same Qwen3-8B int8 weights (exact fp32 image built in {build_s:.1f} s, '
                       f'before timing): {n_tokens} greedy decode steps from position {prompt_len} over a cache whose '
                       f'{prompt_len} slots hold seeded N(0, 1) keys and values (the prefill is not run on the CPU); '
                       f'{dt:.1f} s'),
            'cpu': cpu_name()}


def long_context(prompt_len=8192, steps=32, warmup=4, seed=0, cpu_tokens=0):
    """The long-context workload: a random-init Qwen3-8B-architecture int8 model (36 layers, hidden 4096,
    intermediate 12288, 32 q / 8 kv heads) after a `prompt_len`-token uniform-random prompt, cache of prompt + 512
    slots; `steps` graph replays timed back to back. The step's GEMV launches are timed on their own
    (gemv_roofline); the rest of the step, attention and its merge launches plus the argmax, is the step time minus
    that, over the K/V bytes of the live slots."""
    from efficientgpt_amd.qwen3 import QWEN3_8B, Qwen3Int8Engine
    cfg = QWEN3_8B
    cap = prompt_len + 512
    eng = Qwen3Int8Engine.random(cfg, cap, seed=seed, keep_weights=cpu_tokens > 0)
    prompt = torch.randint(0, cfg.vocab, (prompt_len,), generator=torch.Generator().manual_seed(seed + 1))
    with torch.inference_mode():
        eng.reset()
        t = time.perf_counter()
        eng.prefill(prompt)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t
        eng.capture()
        for _ in range(warmup):
            eng.replay()
        torch.cuda.synchronize()
        e0, e1 = _events()
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            eng.graph.replay()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        roof = gemv_roofline(eng)
    step_ms = wall / steps * 1e3
    mean_len = prompt_len + warmup + (steps + 1) / 2
    kv_bytes = cfg.kv_bytes_per_slot() * mean_len
    rest_ms = step_ms - roof['gemv_ms_per_step']
    wbytes, sbytes = cfg.weight_bytes()
    step_bytes = wbytes + sbytes + kv_bytes
    nsplit = eng.nsplit
    weights = eng.weights if cpu_tokens > 0 else None
    del eng
    torch.cuda.empty_cache()
    cpu = cpu_long_context(cfg, weights, prompt_len, cpu_tokens, host_threads()) if cpu_tokens > 0 else None
    del weights
    return {'workload': f'qwen3-8b int8, {prompt_len}-token prompt, cache {cap} slots, {steps} graph replays',
            'cpu_baseline': cpu,
            'value': round(steps / wall, 2), 'unit': 'tok/s', 'ms_per_step': round(step_ms, 4),
            'prefill_s': round(prefill_s, 3), 'mean_kv_len': mean_len, 'nsplit': nsplit,
            'step_frac': round(step_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            'gemv': {k: roof[k] for k in ('achieved', 'frac', 'launches', 'avg_launch_us', 'gemv_ms_per_step')},
            'attention_and_rest': {'ms_per_step': round(rest_ms, 4), 'kv_bytes': int(kv_bytes),
                                   'achieved': round(kv_bytes / (rest_ms * 1e-3) / 1e9, 1),
                                   'frac': round(kv_bytes / (rest_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}


def cpu_kernels(threads, rows=(1, 2, 4, 8), lengths=(256, 1024, 4096, 16384, 32768)):
    """The reference's CPU-runnable forms of the two kernels on this host, beside the GPU figures:
    - the int8 linear's formula ((x @ W.bf16^T).float() * s).bf16 (research/realmodel/int8_linear.py:97) at every
      per-layer GEMV shape of Qwen3-1.7B and the lm_head, M = 1, 2, 4, 8 rows, median of 20 calls; the exact bf16
      image of W is built once per shape and reused (numerically identical to converting per call);
    - fp32 SDPA of one query per head over L slots, 16 q / 8 kv heads of 128 (the kv heads repeated per group),
      median of 5 calls, at L = 256 ... 32768.
    Bytes are the kernels' algorithmic bytes (N K + 4 N + 2 M K + 2 M N; 4096 L + 8192)."""
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)

    def timed(fn, reps):
        fn()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return sorted(ts)[len(ts) // 2]

    gemv = {}
    for name, n, k in CONFIG1_SHAPES:
        w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        wb = w.to(torch.bfloat16)
        sc = torch.randn(n, generator=g).abs() * 0.02 / 127
        for m in rows:
            x = torch.randn(m, k, generator=g).to(torch.bfloat16)
            t = timed(lambda: ((x @ wb.t()).float() * sc).to(torch.bfloat16), 20)
            nbytes = n * k + 4 * n + 2 * m * k + 2 * m * n
            gemv[f'{m}x{k}->{n}'] = {'shape': name, 'rows': m, 'us': round(t * 1e6, 1),
                                     'achieved_gbps': round(nbytes / t / 1e9, 2)}
        del w, wb
    attn = {}
    hq, hkv, d = 16, 8, 128
    for L in lengths:
        q = torch.randn(1, hq, 1, d, generator=g)
        kv = torch.randn(2, 1, hkv, L, d, generator=g).to(torch.bfloat16).float()
        kk, vv = kv[0].repeat_interleave(hq // hkv, 1), kv[1].repeat_interleave(hq // hkv, 1)
        t = timed(lambda: torch.nn.functional.scaled_dot_product_attention(q, kk, vv), 5)
        attn[str(L)] = {'us': round(t * 1e6, 1), 'achieved_gbps': round((4096 * L + 8192) / t / 1e9, 2)}
    return {'gemv': gemv, 'attention': attn, 'threads': threads,
            'gemv_note': 'bf16 image of the int8 weights built once per shape, then x @ W^T, fp32 scale, bf16'}


def copy_bandwidth(nbytes=1 << 30, reps=10):
    src = torch.empty(nbytes, dtype=torch.uint8, device='cuda')
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = _events()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) / 1e3 / reps
    del src, dst
    torch.cuda.empty_cache()
    return round(2 * nbytes / s / 1e9, 1)  # bytes read + bytes written


def cpu_name():
    """The host CPU's model name from /proc/cpuinfo, as the reference's environment record reads it
    (research/release/collect_env.py:40-45); the platform's processor string where that file has none."""
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def gpu_busy_percent():
    """The GPU's busy percentage from the amdgpu driver (sysfs gpu_busy_percent of the device torch runs on), read
    before timing as the reference reads nvidia-smi's utilisation (research/realmodel/bench_int8.py:46-51); None
    where the file is not readable."""
    try:
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        bus = f'{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:{props.pci_device_id:02x}.0'
        with open(f'/sys/bus/pci/devices/{bus}/gpu_busy_percent') as f:
            return float(f.read().strip())
    except (OSError, AttributeError, ValueError):
        return None


def host_threads():
    """CPU threads this process may use: OMP_NUM_THREADS if set, else the cores in its affinity mask."""
    env = os.environ.get('OMP_NUM_THREADS')
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0)) or 1


def near_tie_bound(top1):
    """Greedy near-tie margin: the reference's 1e-2 on fp32 logits (research/phase5/benchmark_review.py:46),
    or two bf16 ulps of the top logit when that is larger."""
    a = abs(top1)
    return max(1e-2, 2 * 2.0 ** (math.floor(math.log2(a)) - 7) if a > 0 else 0.0)


def cpu_baseline(eng, prompt, n_tokens, gpu_tokens):
    """The CPU oracle on the same weights: prefill the prompt, then greedy tokens until n_tokens are out.
    Decode tok/s = (n - 1) / (total - TTFT), the reference's client-side rule (assistant/backends.py:276,
    research/realmodel/bench_int8.py)."""
    from oracle.qwen3 import Qwen3Oracle, Qwen3Shape
    c = eng.cfg
    torch.set_num_threads(host_threads())
    shape = Qwen3Shape(c.vocab, c.hidden, c.inter, c.layers, c.heads, c.kv_heads, c.head_dim, c.rope_theta,
                       c.rms_eps, c.tied)
    orc = Qwen3Oracle(shape, eng.weights, dtype=torch.bfloat16, cap=len(prompt) + n_tokens + 1)
    orc.forward(prompt[:1], 0)  # builds the cached fp32 images of the int8 weights outside the timed run
    orc.reset()
    margins = []  # (top-1 - top-2, top-1) of the oracle's logits at each step
    logits_at = []  # the oracle's logits at each step (bf16)

    def pick(logits):
        top2 = torch.topk(logits.float(), 2).values
        margins.append((float(top2[0] - top2[1]), float(top2[0])))
        logits_at.append(logits.to(torch.bfloat16))
        return int(torch.argmax(logits))

    t0 = time.perf_counter()
    toks = [pick(orc.forward(prompt, 0))]
    t_first = time.perf_counter()
    pos = len(prompt)
    for _ in range(n_tokens - 1):
        toks.append(pick(orc.forward([toks[-1]], pos)))
        pos += 1
    t1 = time.perf_counter()
    decode_tps = (n_tokens - 1) / (t1 - t_first) if n_tokens > 1 else None
    # Teacher-forced comparison (outside the CPU timing): the GPU step fed the oracle's own tokens, its pick at
    # every step against the oracle's; a disagreement counts as a near-tie when the oracle's top-1 / top-2 margin
    # is at most twice the GPU-oracle logit distance at that step (the reference's rule, widened as below).
    with torch.inference_mode():
        eng.reset()
        got = eng.prefill(prompt)
        tf_agree, tf_ties, tf_dist = 0, 0, 0.0
        for i in range(n_tokens):
            if i:
                eng.token.fill_(toks[i - 1])
                eng.replay()
                got = eng.logits[0]
            g = got.float().cpu()
            dist = float((g - logits_at[i].float()).abs().max())
            tf_dist = max(tf_dist, dist)
            if int(torch.argmax(g)) == toks[i]:
                tf_agree += 1
            elif margins[i][0] <= 2 * dist:
                tf_ties += 1
    teacher_forced = (f'{tf_agree}/{n_tokens} steps pick the oracle\'s token; the other {n_tokens - tf_agree} are '
                      f'near-ties: {tf_ties} of them (oracle margin <= twice the GPU-oracle logit distance, at most '
                      f'{tf_dist:.3g} over the run)')
    gpu = list(gpu_tokens[:n_tokens])
    first = next((i for i, (a, b) in enumerate(zip(toks, gpu)) if a != b), None)
    agree = f'{n_tokens}/{n_tokens} identical'
    if first is not None:  # free-running decodes: after a divergence the contexts differ
        m, top = margins[first]
        bound = near_tie_bound(top)
        # The GPU's logits at that step on the oracle's own tokens (teacher-forced): their distance from the
        # oracle's is this model's rounding noise there. The reference sets its near-tie bound just above the
        # logit noise it measured between two implementations (research/phase5/benchmark_review.py:43-46);
        # the same rule here: a divergence is a near-tie if the margin is at most twice that distance.
        with torch.inference_mode():
            eng.reset()
            got = eng.prefill(prompt)
            for t in toks[:first]:
                eng.token.fill_(t)
                eng.replay()
                got = eng.logits[0]
            dist = float((got.float().cpu() - logits_at[first].float()).abs().max())
        verdict = 'a near-tie' if m <= 2 * dist else 'NOT a near-tie'
        agree = (f'first {first}/{n_tokens} identical; at step {first} the oracle\'s top-1/top-2 margin is {m:.4g} '
                 f'(two bf16 ulps of its top logit: {bound:.4g}), the GPU\'s logits there on the oracle\'s tokens '
                 f'{dist:.4g} from the oracle\'s: {verdict} (margin <= twice that distance)')
    return {'value': round(decode_tps, 3) if decode_tps else None, 'unit': 'tok/s', 'cores': torch.get_num_threads(),
            'kind': 'port',
            'sample': (f'CPU oracle (torch, bf16 activations, exact fp32 image of the int8 weights built before '
                       f'timing) on the same weights and prompt: prefill of the {len(prompt)}-token prompt (TTFT '
                       f'{t_first - t0:.2f} s), then {n_tokens} greedy tokens in {t1 - t0:.1f} s; decode tok/s = '
                       f'(n-1)/(total-TTFT)'),
            'ttft_s': round(t_first - t0, 3), 'total_s': round(t1 - t0, 3), 'tokens': n_tokens,
            'cpu': cpu_name(),
            'token_agreement_with_gpu': agree, 'teacher_forced_agreement': teacher_forced,
            'teacher_forced_agree': tf_agree, 'teacher_forced_near_ties': tf_ties}


def dispatch_grid(inner=20, reps=20):
    """Single pass (1 split) against the default split count of egpt_decode_attn, bf16, every row at position
    cap - 1, 20 calls per captured graph (warm: the point is the launch structure, not HBM). MHA 6 x 64 (the
    reference's Phase-5 shape), and 16 / 8 and 32 / 8 heads at D 128 (Qwen3-1.7B / -8B)."""
    from efficientgpt_amd.decode_attention import decode_attention, decode_attention_single_pass
    for (hq, hkv, d), b, cap in itertools.product([(6, 6, 64), (16, 8, 128), (32, 8, 128)],
                                                   [1, 2, 4, 8, 16, 32, 64, 128], [16, 32, 64, 128, 256, 1024, 4096]):
        q = torch.randn(b, hq, 1, d, device='cuda', dtype=torch.bfloat16)
        k = torch.randn(b, hkv, cap, d, device='cuda', dtype=torch.bfloat16)
        v = torch.randn_like(k)
        pos = torch.full((b,), cap - 1, device='cuda', dtype=torch.long)

        def many(fn):
            return lambda: [fn() for _ in range(inner)]
        t1 = min(_time_graph(many(lambda: decode_attention_single_pass(q, k, v, pos)), reps) for _ in range(3))
        ts = min(_time_graph(many(lambda: decode_attention(q, k, v, pos)), reps) for _ in range(3))
        print(json.dumps({'hq': hq, 'hkv': hkv, 'd': d, 'batch': b, 'cap': cap,
                          'single_pass_us': round(t1 / inner * 1e6, 2), 'default_us': round(ts / inner * 1e6, 2)}),
              flush=True)
        del q, k, v


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({'error': 'bench.py measures one GPU; runs on several GPUs are not supported',
                          'n_gpus': args.gpus}), flush=True)
        sys.exit(2)
    if args.dispatch_grid:
        torch.cuda.set_device(0)
        dispatch_grid()
        return
    if args.attention_only:
        torch.cuda.set_device(0)
        hq, hkv = (int(v) for v in args.heads.split('/'))
        with torch.inference_mode():
            for L in (int(v) for v in args.attention_only.split(',')):
                r = attention_roofline(L=L, hq=hq, hkv=hkv, copies=max(4, (1 << 29) // (4096 * L) + 1), reps=5)
                r['heads'] = f'{hq}/{hkv}'
                print(json.dumps(r), flush=True)
        return
    from efficientgpt_amd.fast_decode import GraphGreedyDecoder
    from efficientgpt_amd.qwen3 import QWEN3_1_7B, QWEN3_8B, Qwen3Int8Engine

    cfg = QWEN3_1_7B if args.model == 'qwen3-1.7b' else QWEN3_8B
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    busy_at_start = gpu_busy_percent()  # before this process runs anything on the GPU
    n_stream = 256 if args.model == 'qwen3-1.7b' else 64
    cap = args.prompt + max(args.warmup + args.steps, n_stream) + 8
    t = time.perf_counter()
    want_cpu = args.cpu_tokens > 0 and args.model == 'qwen3-1.7b'
    eng = Qwen3Int8Engine.random(cfg, cap, seed=args.seed, device=dev, keep_weights=want_cpu)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t
    prompt = torch.randint(0, cfg.vocab, (args.prompt,), generator=torch.Generator().manual_seed(args.seed + 1))

    with torch.inference_mode():
        # GPU decode: prefill, capture, warm-up replays, then K timed replays back to back
        eng.reset()
        t = time.perf_counter()
        eng.prefill(prompt)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t
        eng.capture()
        # Rounds of the same workload: each restores the token and position the prefill left (the cache past the
        # prompt is rewritten by the round's own steps), replays W warm-up steps, then times K steps.
        token0, pos0 = eng.token.clone(), eng.position.clone()
        rounds = []
        for _ in range(max(1, args.rounds)):
            eng.token.copy_(token0)
            eng.position.copy_(pos0)
            for _ in range(args.warmup):
                eng.replay()
            torch.cuda.synchronize()
            e0, e1 = _events()
            t0 = time.perf_counter()
            e0.record()
            for _ in range(args.steps):
                eng.graph.replay()
            e1.record()
            torch.cuda.synchronize()
            rounds.append((time.perf_counter() - t0, e0.elapsed_time(e1) / 1e3))
        walls = sorted(r[0] for r in rounds)
        wall = walls[len(walls) // 2]  # the median round (lower median for an even count)
        gpu_s = sorted(r[1] for r in rounds)[len(rounds) // 2]
        value = args.steps / wall
        rounds_rec = {'rounds': len(rounds), 'steps_per_round': args.steps,
                      'tok_s': [round(args.steps / r[0], 2) for r in rounds],
                      'median': round(value, 2), 'min': round(args.steps / walls[-1], 2),
                      'max': round(args.steps / walls[0], 2),
                      'gpu_busy_percent_at_start': busy_at_start,
                      'contended': None if busy_at_start is None else busy_at_start > 10.0}
        mean_len = args.prompt + args.warmup + (args.steps + 1) / 2

        roof = gemv_roofline(eng)
        roof['traffic'] = measured_traffic(args.model)
        if roof['traffic'] is not None:
            roof['traffic_source'] = ('rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of bench.py, scaled by a 1 GiB copy: '
                                      'profiles/fused_gemv_traffic_qwen3_1p7b.md')

        stream = None
        gpu_tokens = []
        if not args.no_stream:
            dec = GraphGreedyDecoder(eng, max_cache_len=cap)
            out, st = dec.generate(prompt.view(1, -1).to(dev), n_stream)
            gpu_tokens = out
            stream = {'decode_tok_s': round((st['tokens'] - 1) / (st['total_s'] - st['ttft_s']), 2),
                      'ttft_ms': round(st['ttft_s'] * 1e3, 2), 'tokens': st['tokens'],
                      'distinct_tokens': len(set(out))}
    extra = {}
    if not args.no_extra:
        with torch.inference_mode():  # graph capture after the engine's inference-mode captures
            floor = launch_floor()
            extra['launch_floor_us'] = floor
            extra['attention'] = attention_roofline()
            extra['attention_by_length'] = attention_sweep()
            extra['gemv_1x2048_6144'] = gemv_cfg0()
            # each small kernel's own share: its bytes over its time less the launch floor (one per launch)
            g0 = extra['gemv_1x2048_6144']
            g0['frac_beyond_floor'] = round(g0['bytes_per_call'] / max(g0['us_per_call'] - floor, 1e-3) / 1e3
                                            / HBM_PEAK_GBPS, 4)
            # the dominant kernel family likewise: the step's GEMV launches less one floor each
            roof['frac_beyond_floor'] = round(
                roof['bytes_per_step'] / max(roof['gemv_ms_per_step'] * 1e3 - roof['launches'] * floor, 1e-3)
                / 1e3 / HBM_PEAK_GBPS, 4)
            for L, r in list(extra['attention_by_length'].items()) + [('32768', extra['attention'])]:
                launches = 1 if r['nsplit'] == 1 else 2  # the split kernel, then the combine
                r['frac_beyond_floor'] = round((4096 * int(L) + 8192) / max(r['us_per_call'] - launches * floor, 1e-3)
                                               / 1e3 / HBM_PEAK_GBPS, 4)
            extra['gemv_small_batch'] = gemv_small_batch(floor)
            extra['gemv_reference_shapes'] = gemv_reference_shapes()
            extra['prefill_gemm'] = prefill_gemm()
            extra['copy_gbps'] = copy_bandwidth()
    if args.model == 'qwen3-1.7b' and not args.no_long_context:
        extra['long_context'] = long_context(cpu_tokens=args.cpu_long_tokens)
    cpu = None
    if args.cpu_tokens > 0 and gpu_tokens and args.model == 'qwen3-1.7b':
        cpu = cpu_baseline(eng, prompt, args.cpu_tokens, gpu_tokens)
        cpu['kernels'] = cpu_kernels(cpu['cores'])

    wbytes, sbytes = cfg.weight_bytes()
    step_bytes = wbytes + sbytes + cfg.kv_bytes_per_slot() * mean_len + 2 * cfg.hidden
    step_s = wall / args.steps
    line = {
        'metric': 'batch-1 decode tok/s (Qwen3-%s-shape int8); GEMV/attn HBM GB/s vs peak'
                  % ('1.7B' if args.model == 'qwen3-1.7b' else '8B'),
        'value': round(value, 2), 'unit': 'tok/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': round(step_s * 1e3, 4), 'gpu_ms_per_step': round(gpu_s / args.steps * 1e3, 4),
        'spread': rounds_rec, 'host_cpu': cpu_name(),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'int8',
        'data': 'synthetic: random-init weights N(0,0.02), uniform-random prompt ids',
        'config': {'workload': f'{args.model} int8 weight-only batch-1 greedy decode, {args.prompt}-token prompt, '
                               f'one graph replay per token (int8 weights, bf16 activations, fp32 accumulation)',
                   'model': args.model, 'global_batch': 1, 'seq_len': args.prompt + args.warmup + args.steps,
                   'parallelism': 'single GPU'},
        'roofline': roof,
        'cpu_baseline': cpu,
        'step': {'bytes': int(step_bytes), 'achieved_gbps': round(step_bytes / step_s / 1e9, 1),
                 'frac': round(step_bytes / step_s / 1e9 / HBM_PEAK_GBPS, 4), 'mean_kv_len': mean_len,
                 'launches': cfg.layers * (5 if eng.nsplit <= 16 else 6) + 2,
                 'form': 'fused, one launch per phase (egpt_qwen3_decode_step)'},
        'prefill_s': round(prefill_s, 3),
        'streamed_generate': stream,
        # The reference's own published rate for this decode (other hardware; vs_baseline stays null since no
        # MI355X figure exists): Qwen3-1.7B int8 with its CUDA-graph decoder, batch 1, 256 new tokens
        # (the reference's README.md:32-37, BENCHMARK_REPORT.md:22-29).
        'reference_published': ({'value': 111.9, 'unit': 'tok/s', 'hardware': 'NVIDIA RTX 4060',
                                 'ratio': round(value / 111.9, 2)} if args.model == 'qwen3-1.7b' else None),
        'build_s': round(build_s, 1),
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
