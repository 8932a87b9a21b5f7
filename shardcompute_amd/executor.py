"""Inference executor: prompt prefill and token generation on one GPU.

Drop-in for ``ParallelExecutor`` of ``src/shardcompute/worker/executor.py:67-373``
(``forward``, ``forward_with_timing``, ``generate``, ``reset_cache``,
``get_metrics``, ``get_timing_summary``, and the ``ExecutionMetrics`` /
``LayerTiming`` records).

Greedy generation (``temperature == 0``, ``executor.py:267-325``) never
synchronises with the host per token.  The prompt is prefilled eagerly into a
preallocated :class:`~shardcompute_amd.kv_cache.KVCache`; one decode step
(embed -> layers -> norm -> lm_head -> argmax -> counter advance) runs eagerly
once, is then captured in a HIP graph (``torch.cuda.CUDAGraph``), and the graph
is replayed once per further token.  Positions, the cache length and the output
slot are device counters, so the same graph serves every step.  Stop tokens are
checked on the host every ``check_every`` tokens; tokens generated past a stop
token are discarded, so the output matches a per-token check.

Sampling (``temperature > 0``: temperature, top-p, categorical draw, as in
``executor.py:280-305``) runs eagerly with torch ops on the device and is not
part of the measured greedy path.
"""
import time
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional

import torch

from . import _lib
from .decode_plan import maybe_plan
from .kv_cache import KVCache, round_capacity
from .parallel.transformer import ParallelTransformer, StepBuffers, run_sync


@dataclass
class LayerTiming:
    layer_idx: int
    layer_type: str = "transformer"     # "embedding", "transformer", "lm_head"
    compute_ms: float = 0.0
    comm_ms: float = 0.0

    @property
    def total_ms(self) -> float:
        return self.compute_ms + self.comm_ms


@dataclass
class ExecutionMetrics:
    total_time_ms: float
    layer_timings: List[LayerTiming] = field(default_factory=list)
    input_tokens: int = 0
    output_shape: List[int] = field(default_factory=list)

    @property
    def compute_time_ms(self) -> float:
        return sum(t.compute_ms for t in self.layer_timings)

    @property
    def comm_time_ms(self) -> float:
        return sum(t.comm_ms for t in self.layer_timings)

    @property
    def compute_fraction(self) -> float:
        tot = self.compute_time_ms + self.comm_time_ms
        return self.compute_time_ms / tot if tot > 0 else 1.0

    def to_dict(self) -> Dict[str, Any]:
        return {
            "total_time_ms": self.total_time_ms,
            "compute_time_ms": self.compute_time_ms,
            "comm_time_ms": self.comm_time_ms,
            "compute_fraction": self.compute_fraction,
            "input_tokens": self.input_tokens,
            "output_shape": self.output_shape,
            "num_layers": len([t for t in self.layer_timings if t.layer_type == "transformer"]),
            "layer_timings": [{"layer": t.layer_idx, "type": t.layer_type, "compute_ms": t.compute_ms,
                               "comm_ms": t.comm_ms} for t in self.layer_timings],
        }


TokenCallback = Callable[[int, int, bool], Any]


class DecodeGraph:
    """Greedy decode steps of ``model`` for ``batch`` sequences, as replayable graphs:
    one of a single step and one of ``steps_per_graph`` consecutive steps.  Every
    step reads its position and token column from device counters, so a graph
    replays unchanged at any position; the longer graph pays the start and end of
    a graph launch once per ``steps_per_graph`` steps instead of once per step."""

    def __init__(self, model: ParallelTransformer, cache: KVCache, tokens: torch.Tensor, use_graph: bool = True,
                 fused_trunk: bool = True, steps_per_graph: int = 8):
        self.model = model
        self.cache = cache
        self.tokens = tokens
        self.bufs = StepBuffers(model, cache.batch, 1, cache.capacity)
        if fused_trunk:
            self.bufs.plan = maybe_plan(model, cache, self.bufs.ids, self.bufs.h)
        self.use_graph = use_graph
        self.steps_per_graph = max(1, int(steps_per_graph))
        self.graph = None           # (graph, logits of its step)
        self.graph_n = None         # (graph, logits of its last step)
        self.logits = None          # logits of the most recent step

    def _step(self):
        self.logits = self.model.decode_step(self.bufs, self.cache, self.tokens)

    def run(self, n: int):
        """Advance ``n`` tokens (the first call runs one step eagerly, then captures)."""
        S = self.steps_per_graph
        while n > 0:
            if self.graph is not None and S > 1 and n >= S:
                self.cache.check_room(S)
                if self.graph_n is None:
                    self.graph_n = self._capture(S)
                g, self.logits = self.graph_n
                g.replay()
                self.cache.length += S
                n -= S
                continue
            self.cache.check_room(1)
            if self.graph is not None:
                g, self.logits = self.graph
                g.replay()
            else:
                self._step()
                if self.use_graph:
                    eager = self.logits
                    self.graph = self._capture(1)
                    # capture only records: the step's logits are the eager run's
                    self.logits = eager
            self.cache.length += 1
            n -= 1

    def _capture(self, steps: int):
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(steps):
                self._step()
        return g, self.logits


class ParallelExecutor:
    def __init__(self, rank: int, world_size: int, communicator, model: ParallelTransformer, *,
                 use_graphs: bool = True, check_every: int = 16):
        self.rank = rank
        self.world_size = world_size
        self.communicator = communicator
        self.model = model
        self.use_graphs = use_graphs
        self.check_every = max(1, int(check_every))
        self.last_metrics: Optional[ExecutionMetrics] = None
        self._past_key_values: Optional[KVCache] = None

    # ---------------------------------------------------------------- forward

    def _ensure_cache(self, batch: int, needed: int, exact: bool = False) -> KVCache:
        """A cache with room for ``needed`` more positions.

        The reference's cache grows by one concatenation per step; here a cache
        that is too small is replaced by one with room for the cached positions
        plus ``needed`` (doubled, unless ``exact``: ``generate`` knows its final
        length), and the cached positions are copied over.  The capacity never
        defaults to ``max_position_embeddings``: a Llama-3 config's 8 K or 128 K
        positions would reserve gigabytes per sequence and make the batch-1
        decode plan's attention state exceed a CU's LDS."""
        c = self._past_key_values
        if c is not None and c.batch != batch:
            c = None
        have = 0 if c is None else c.length
        if c is None or c.capacity < have + needed:
            want = have + needed
            if not exact and c is not None:
                want = max(want, 2 * c.capacity)
            newc = self.model.new_cache(batch, round_capacity(want))
            if c is not None and c.length:
                newc.load_tuples(c.as_tuples())
            self._past_key_values = c = newc
        return c

    async def forward(self, input_ids, attention_mask=None, use_cache: bool = False, *, last_only: bool = False):
        t0 = time.perf_counter()
        ids = torch.as_tensor(input_ids).to(self.model.device)
        cache = self._ensure_cache(ids.shape[0], ids.shape[1]) if use_cache else None
        logits, _ = await self.model.forward(ids, attention_mask=attention_mask, past_key_values=cache,
                                             use_cache=use_cache, last_only=last_only)
        torch.cuda.synchronize()
        self.last_metrics = ExecutionMetrics(total_time_ms=(time.perf_counter() - t0) * 1000,
                                             input_tokens=int(ids.numel()), output_shape=list(logits.shape))
        return logits

    async def forward_with_timing(self, input_ids, attention_mask=None):
        """A cache-less forward with each stage timed on the GPU
        (``worker/executor.py:155-227``): the embedding (layer -1), every
        transformer block, and the final norm + lm_head (layer -2).

        Each stage is bracketed by HIP events on the current stream, so its
        ``compute_ms`` is the stage's own GPU time (the reference times each
        stage with ``mx.eval`` and the host clock).  There are no collectives on
        one GPU: ``comm_ms`` is 0.  Returns ``(logits, metrics)``."""
        m = self.model
        t0 = time.perf_counter()
        ids = torch.as_tensor(input_ids).to(m.device)
        B, S = ids.shape
        ev = [torch.cuda.Event(enable_timing=True)]
        ev[0].record()
        h = await m.embed_tokens.forward(ids)
        ev.append(torch.cuda.Event(enable_timing=True))
        ev[-1].record()
        for layer in m.layers:
            h, _ = await layer.forward(h, attention_mask)
            ev.append(torch.cuda.Event(enable_timing=True))
            ev[-1].record()
        logits = await m._head(h.reshape(B * S, m.hidden_size), None, B, S, False)
        ev.append(torch.cuda.Event(enable_timing=True))
        ev[-1].record()
        torch.cuda.synchronize()
        span = [ev[i].elapsed_time(ev[i + 1]) for i in range(len(ev) - 1)]
        timings = [LayerTiming(-1, "embedding", span[0])]
        timings += [LayerTiming(i, "transformer", span[1 + i]) for i in range(len(m.layers))]
        timings.append(LayerTiming(-2, "lm_head", span[-1]))
        logits = logits.reshape(B, S, -1)
        self.last_metrics = ExecutionMetrics(total_time_ms=(time.perf_counter() - t0) * 1000, layer_timings=timings,
                                             input_tokens=int(ids.numel()), output_shape=list(logits.shape))
        return logits, self.last_metrics

    # ---------------------------------------------------------------- generation

    def _sample(self, logits, temperature, top_p):
        probs = torch.softmax(logits.float() / temperature, dim=-1)
        sp, si = torch.sort(probs, dim=-1, descending=True)
        cum = torch.cumsum(sp, dim=-1)
        keep = cum <= top_p
        keep = torch.cat([torch.ones_like(keep[:, :1]), keep[:, :-1]], dim=-1)
        sp = torch.where(keep, sp, torch.zeros_like(sp))
        sp = sp / sp.sum(dim=-1, keepdim=True)
        pick = torch.multinomial(sp, 1)
        return torch.gather(si, -1, pick)[:, 0].to(torch.int32)

    async def generate(self, input_ids, max_new_tokens: int = 100, temperature: float = 0.7, top_p: float = 0.9,
                       stop_tokens: Optional[List[int]] = None, token_callback: Optional[TokenCallback] = None):
        stop = set(stop_tokens or [])
        t0 = time.perf_counter()
        ids = torch.as_tensor(input_ids).to(self.model.device)
        out_dtype = ids.dtype
        B, S = ids.shape
        self._past_key_values = None
        cache = self._ensure_cache(B, S + max(1, max_new_tokens), exact=True)
        cache.reset()
        if max_new_tokens <= 0:
            return ids
        logits, _ = await self.model.forward(ids, past_key_values=cache, use_cache=True, last_only=True)
        tokens = torch.zeros((B, max_new_tokens), dtype=torch.int32, device=ids.device)
        n_done = 0
        emitted = 0

        async def flush(upto):
            # report tokens [emitted, upto) of row 0; return the end position at a stop token
            nonlocal emitted
            if upto <= emitted:
                return None
            host = tokens[0, emitted:upto].tolist()
            for j, tok in enumerate(host):
                idx = emitted + j
                is_stop = tok in stop
                last = is_stop or idx == max_new_tokens - 1
                if token_callback is not None:
                    await token_callback(int(tok), idx, last)
                if is_stop:
                    emitted = idx + 1
                    return idx + 1
            emitted = upto
            return None

        if temperature == 0:
            dec = DecodeGraph(self.model, cache, tokens, use_graph=self.use_graphs)
            plan = dec.bufs.plan
            # which decode path ran: "trunk" (one launch per token) or "per-op"
            self.last_decode_path = "trunk" if plan is not None else "per-op"

            def check_plan():
                # the whole-trunk launch bounds every wait; one that gave up left its
                # outputs invalid, and the tokens after it would be silently wrong
                if plan is not None and plan.status() != 0:
                    raise RuntimeError(f"whole-trunk decode launch gave up waiting (status {plan.status()}): "
                                       f"another kernel held CUs it needs; the generated tokens are invalid")

            _lib.argmax(logits.reshape(B, -1), ids=dec.bufs.ids.view(-1), tokens=tokens, step=cache.counters[1:])
            _lib.add_i32(cache.counters[1:], 1, n=1)
            n_done = 1
            end = None
            # tokens reach the host (stop check, streaming callback) every check_every tokens
            report = bool(stop) or token_callback is not None
            while end is None:
                if n_done >= max_new_tokens:
                    check_plan()
                    end = await flush(max_new_tokens) or max_new_tokens
                    break
                if report and n_done - emitted >= self.check_every:
                    check_plan()
                    end = await flush(n_done)
                    if end is not None:
                        break
                chunk = min(self.check_every - (n_done - emitted) if report else self.check_every,
                            max_new_tokens - n_done)
                dec.run(max(1, chunk))
                n_done += max(1, chunk)
            n_gen = end
        else:
            n_gen = None
            nxt = self._sample(logits.reshape(B, -1), temperature, top_p)
            for t in range(max_new_tokens):
                tokens[:, t] = nxt
                end = await flush(t + 1)
                if end is not None or t == max_new_tokens - 1:
                    n_gen = t + 1
                    break
                logits, _ = await self.model.forward(nxt.view(B, 1), past_key_values=cache, use_cache=True)
                nxt = self._sample(logits.reshape(B, -1), temperature, top_p)
        torch.cuda.synchronize()
        self.last_metrics = ExecutionMetrics(total_time_ms=(time.perf_counter() - t0) * 1000, input_tokens=n_gen,
                                             output_shape=[1, n_gen])
        return torch.cat([ids, tokens[:, :n_gen].to(out_dtype)], dim=1)

    def reset_cache(self):
        self._past_key_values = None

    def get_metrics(self) -> Optional[Dict[str, Any]]:
        return self.last_metrics.to_dict() if self.last_metrics else None

    def get_timing_summary(self) -> Dict[str, Any]:
        m = self.last_metrics
        if not m:
            return {}
        return {
            "total_ms": m.total_time_ms,
            "compute_ms": m.compute_time_ms,
            "comm_ms": m.comm_time_ms,
            "compute_fraction": m.compute_fraction,
            "tokens_per_second": m.input_tokens / (m.total_time_ms / 1000) if m.total_time_ms > 0 else 0.0,
        }
