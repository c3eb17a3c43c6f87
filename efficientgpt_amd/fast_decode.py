"""Sync-free greedy decoding: one captured graph replay per token, tokens streamed through pinned memory.

Drop-in for research/realmodel/fast_decode.py: `GraphGreedyDecoder(model,
max_cache_len, lookahead=8)` and `.generate(input_ids, max_new_tokens, eos_ids=(),
on_token=None) -> (tokens, stats)` keep the reference's names, guards (ValueError),
stats keys and streaming semantics (:66-111): every step's token reaches pinned
host memory behind an event (the step's last kernel stores it to the engine's
token ring, so no copy is launched per token), a token is handed out as soon as its
event has fired, the host never waits on the step it has just launched unless more than
`lookahead` steps are in flight, EOS stops the run at (and including) the EOS token,
and tokens that steps launched ahead of it computed are never handed out.

`model` is a Qwen3Int8Engine or a transformers Qwen3 model whose linears are int8
(`quantize_model(model)`, which the reference's HFBackend runs for quant='int8'
before it builds its decoder, assistant/backends.py:200-202, 241). A model with
float linears is refused: the engine runs the int8 contract only, and quantising
behind the caller's back would change the tokens the caller asked for.
`quantize=True` opts in to that. The device step is the engine's captured graph:
embedding through argmax and the token / position update, with no host
synchronisation.

Capacity buckets (assistant/backends.py:162-167, 221-249): `pick_bucket`,
`GRAPH_BUCKETS` and `MAX_GRAPH_DECODERS` keep the reference's names and rule (the
smallest bucket at or under the limit that holds prompt + new tokens, then the
limit itself), and `DecoderPool` keeps one graph decoder per bucket in use, the
least recently used dropped first. Here the buckets share one set of weight tensors
(`Qwen3Int8Engine.with_capacity`); only caches, state and graphs are per bucket.
Graph decoders built one per bucket from the same transformers model, as the
reference's HFBackend does, share them too (`engine_for`).
"""

import collections
import time
import weakref

import torch

from .qwen3 import Qwen3Int8Engine

# Engines taken over from a transformers model, per model: the first one owns the weight tensors, and
# decoders of other capacities get engines sharing them (Qwen3Int8Engine.with_capacity). An engine
# lives while a decoder holds it; the weight owner lives as long as the model.
_MODEL_ENGINES = weakref.WeakKeyDictionary()  # model -> (weight owner, {capacity: engine, weakly held})


def engine_for(model, max_cache_len, quantize=False):
    """The engine of `max_cache_len` slots over a transformers model's int8 weights, sharing them with every
    other engine built from the same model (see Qwen3Int8Engine.from_hf for `quantize`)."""
    entry = _MODEL_ENGINES.get(model)
    if entry is None:
        owner = Qwen3Int8Engine.from_hf(model, max_cache_len, quantize=quantize)
        entry = (owner, weakref.WeakValueDictionary())
        entry[1][owner.cap] = owner
        _MODEL_ENGINES[model] = entry
    owner, by_cap = entry
    eng = by_cap.get(int(max_cache_len))
    if eng is None:
        eng = owner.with_capacity(max_cache_len)
        by_cap[eng.cap] = eng
    return eng


class GraphGreedyDecoder:
    def __init__(self, model, max_cache_len, lookahead=8, quantize=False):
        if isinstance(model, Qwen3Int8Engine):
            if model.cap < max_cache_len:
                raise ValueError('engine cache is smaller than max_cache_len')
            self.engine = model
        else:
            self.engine = engine_for(model, max_cache_len, quantize=quantize)
        self.model = model
        self.max_cache_len, self.lookahead = int(max_cache_len), int(lookahead)
        self.device = self.engine.device
        self.host = torch.empty(self.max_cache_len, dtype=torch.long, pin_memory=True)

    @property
    def graph(self):
        return self.engine.graph

    def _check_request(self, input_ids, max_new_tokens):
        if input_ids.dim() != 2 or input_ids.shape[0] != 1:
            raise ValueError('GraphGreedyDecoder supports batch size 1')
        if max_new_tokens < 1:
            raise ValueError('max_new_tokens must be >= 1')
        if input_ids.shape[1] < 1:
            raise ValueError('prompt must hold at least one token')
        if input_ids.shape[1] + max_new_tokens > self.max_cache_len:
            raise ValueError('prompt + max_new_tokens exceeds max_cache_len')

    @torch.inference_mode()
    def generate(self, input_ids, max_new_tokens, eos_ids=(), on_token=None):
        self._check_request(input_ids, max_new_tokens)
        eng = self.engine
        capture_s = 0.0
        if eng.graph is None:  # first request: capture the step (timed apart from TTFT)
            t = time.perf_counter()
            eng.capture()
            capture_s = time.perf_counter() - t
        eng.reset()
        stop = frozenset(int(e) for e in eos_ids)
        tokens, t_first = [], None
        # (pinned host tensor, slot, event after which the slot holds the token), oldest first
        in_flight = collections.deque()
        # With the engine's token ring, each replay stores its token to pinned memory itself (no copy launched
        # per token): token k of the request lands at ring slot (prompt length + k) % capacity.
        ring = eng.token_ring if getattr(eng, '_ring_dev', None) else None
        plen = int(input_ids.shape[1])
        t0 = time.perf_counter()
        eng.prefill(input_ids[0])  # the first new token is now in eng.token
        for step in range(max_new_tokens):
            if step == 0 or ring is None:
                self.host[step:step + 1].copy_(eng.token, non_blocking=True)
                copied = torch.cuda.Event()
                copied.record()
                in_flight.append((self.host, step, copied))
            final = step + 1 == max_new_tokens
            if not final:
                eng.graph.replay()  # overwrites eng.token with the next step's pick
                if ring is not None:
                    stored = torch.cuda.Event()
                    stored.record()
                    in_flight.append((ring, (plen + step + 1) % eng.cap, stored))
            # hand out what has landed; block only to keep the run-ahead within the lookahead, or at the end
            while in_flight and (final or len(in_flight) > self.lookahead or in_flight[0][2].query()):
                buf, slot, copied = in_flight.popleft()
                copied.synchronize()
                tok = int(buf[slot])
                if t_first is None:
                    t_first = time.perf_counter()
                tokens.append(tok)
                if on_token:
                    on_token(tok)
                if tok in stop:
                    in_flight.clear()
                    break
            if tokens and tokens[-1] in stop:
                break
        torch.cuda.synchronize(self.device)
        total = time.perf_counter() - t0
        return tokens, {'ttft_s': t_first - t0, 'total_s': total, 'tokens': len(tokens), 'capture_s': capture_s}


# The reference's graph capacity buckets and pool size (assistant/backends.py:221-222).
GRAPH_BUCKETS = (256, 384, 512, 1024, 2048, 4096)
MAX_GRAPH_DECODERS = 3


def pick_bucket(need, buckets, limit):
    """Smallest cache capacity >= need among the buckets at or under `limit`, then `limit` itself; None if the
    request does not fit (assistant/backends.py:162-167)."""
    for c in sorted(b for b in buckets if b <= limit) + [limit]:
        if c >= need:
            return c
    return None


class DecoderPool:
    """Graph decoders over one model, one per capacity bucket in use (assistant/backends.py:232-249).

    `generate(input_ids, max_new_tokens, ...)` runs the request on the decoder of the smallest bucket that holds
    prompt + max_new_tokens, capturing its graph on first use; at most `max_decoders` are kept, the least recently
    used dropped first. Every bucket's engine shares the weight tensors of the first one. Stats are the
    decoder's, plus `capacity` (the bucket) and `capture_s` including a new decoder's construction.
    """

    def __init__(self, model, limit=GRAPH_BUCKETS[-1], buckets=GRAPH_BUCKETS, max_decoders=MAX_GRAPH_DECODERS,
                 lookahead=8, quantize=False):
        if limit < 1:
            raise ValueError('limit must be >= 1')
        if max_decoders < 1:
            raise ValueError('max_decoders must be >= 1')
        self.model, self.limit, self.buckets = model, int(limit), tuple(int(b) for b in buckets)
        self.max_decoders, self.lookahead = int(max_decoders), int(lookahead)
        self.quantize = bool(quantize)
        self.base = model if isinstance(model, Qwen3Int8Engine) else None  # a transformers model: engine_for()
        self.decoders = {}  # capacity -> GraphGreedyDecoder, least recently used first

    def capacity_for(self, need):
        cap = pick_bucket(need, self.buckets, self.limit)
        if cap is None:
            raise ValueError('No capacity bucket large enough for request')
        return cap

    def decoder(self, need):
        """The decoder for a request of `need` cache slots (built on first use) and its construction time."""
        cap = self.capacity_for(need)
        build_s = 0.0
        if cap not in self.decoders:
            while len(self.decoders) >= self.max_decoders:
                del self.decoders[next(iter(self.decoders))]
                torch.cuda.empty_cache()
            t = time.perf_counter()
            if self.base is None:
                engine = engine_for(self.model, cap, quantize=self.quantize)
            elif self.base.cap == cap and not any(d.engine is self.base for d in self.decoders.values()):
                engine = self.base
            else:
                engine = self.base.with_capacity(cap)
            self.decoders[cap] = GraphGreedyDecoder(engine, cap, lookahead=self.lookahead)
            build_s = time.perf_counter() - t
        dec = self.decoders.pop(cap)
        self.decoders[cap] = dec  # most recently used
        return dec, build_s

    def generate(self, input_ids, max_new_tokens, eos_ids=(), on_token=None):
        if input_ids.dim() != 2 or input_ids.shape[0] != 1:
            raise ValueError('DecoderPool supports batch size 1')
        if max_new_tokens < 1:
            raise ValueError('max_new_tokens must be >= 1')
        dec, build_s = self.decoder(input_ids.shape[1] + max_new_tokens)
        out, st = dec.generate(input_ids, max_new_tokens, eos_ids=eos_ids, on_token=on_token)
        st['capture_s'] = build_s + st.get('capture_s', 0.0)
        st['capacity'] = dec.max_cache_len
        return out, st
