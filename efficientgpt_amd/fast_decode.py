"""Sync-free greedy decoding: one captured graph replay per token, tokens streamed through pinned memory.

Drop-in for research/realmodel/fast_decode.py: `GraphGreedyDecoder(model,
max_cache_len, lookahead=8)` and `.generate(input_ids, max_new_tokens, eos_ids=(),
on_token=None) -> (tokens, stats)` keep the reference's names, guards (ValueError),
stats keys and host-loop semantics (:66-111): each step enqueues a non-blocking copy
of its token into pinned host memory and records an event; the host emits every
token whose event has completed, never blocking on the step it just launched; the
run-ahead is bounded by `lookahead`, EOS stops emission at (and including) the EOS
token, and run-ahead tokens past it are never emitted.

`model` is a Qwen3Int8Engine or a transformers Qwen3 model (its weights are taken
over by an engine; int8 linears as they are, float linears quantised per output
channel). The device step is the engine's captured graph: embedding through argmax
and the token / position update, with no host synchronisation.
"""

import time

import torch

from .qwen3 import Qwen3Int8Engine


class GraphGreedyDecoder:
    def __init__(self, model, max_cache_len, lookahead=8):
        if isinstance(model, Qwen3Int8Engine):
            if model.cap < max_cache_len:
                raise ValueError('engine cache is smaller than max_cache_len')
            self.engine = model
        else:
            self.engine = Qwen3Int8Engine.from_hf(model, max_cache_len)
        self.model = model
        self.max_cache_len, self.lookahead = int(max_cache_len), int(lookahead)
        self.device = self.engine.device
        self.host = torch.empty(self.max_cache_len, dtype=torch.long, pin_memory=True)

    @property
    def graph(self):
        return self.engine.graph

    @torch.inference_mode()
    def generate(self, input_ids, max_new_tokens, eos_ids=(), on_token=None):
        if input_ids.dim() != 2 or input_ids.shape[0] != 1:
            raise ValueError('GraphGreedyDecoder supports batch size 1')
        p = input_ids.shape[1]
        if max_new_tokens < 1:
            raise ValueError('max_new_tokens must be >= 1')
        if p < 1:
            raise ValueError('prompt must hold at least one token')
        if p + max_new_tokens > self.max_cache_len:
            raise ValueError('prompt + max_new_tokens exceeds max_cache_len')
        eng = self.engine
        capture_s = 0.0
        if eng.graph is None:
            t = time.perf_counter()
            eng.capture()
            capture_s = time.perf_counter() - t  # reported separately, not inside TTFT
        eng.reset()
        eos = set(int(e) for e in eos_ids)
        t0 = time.perf_counter()
        eng.prefill(input_ids[0])  # leaves the first new token in eng.token, position = p
        events, out, emitted, first, launched, done = [], [], 0, None, 0, False
        while not done:
            self.host[launched:launched + 1].copy_(eng.token, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            events.append(ev)
            launched += 1
            if launched < max_new_tokens:
                eng.graph.replay()  # computes the next token into eng.token
            while emitted < launched and (events[emitted].query() or launched - emitted > self.lookahead
                                          or launched >= max_new_tokens):
                events[emitted].synchronize()
                tok = int(self.host[emitted])
                if tok < 0:  # the persistent step's failure mark
                    eng.check_status()
                    raise RuntimeError('decode step reported a failure')
                if first is None:
                    first = time.perf_counter()
                out.append(tok)
                if on_token:
                    on_token(tok)
                emitted += 1
                if tok in eos:
                    done = True
                    break
            if launched >= max_new_tokens and emitted >= launched:
                done = True
        torch.cuda.synchronize(self.device)
        total = time.perf_counter() - t0
        return out, {'ttft_s': first - t0, 'total_s': total, 'tokens': len(out), 'capture_s': capture_s}
