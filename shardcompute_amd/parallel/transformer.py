"""Decoder stack over the HIP kernels (one rank's shard).

Drop-in for ``src/shardcompute/parallel/transformer.py``: ``RMSNorm``
(``:17-61``), ``ParallelTransformerBlock`` (``:64-336``) and
``ParallelTransformer`` (``:339-596``) keep their constructor arguments,
loaders, attributes and ``async forward`` signatures.

``ParallelTransformer.forward`` runs a layer as four quantized products plus
RoPE/append and attention: RMSNorm(h + pending) inside the fused q|k|v product,
RoPE/KV append, attention, o_proj, RMSNorm(h + o) inside the fused gate|up
product whose kernel also applies silu(gate) * up to paired columns, and
down_proj.  The residual adds of
``transformer.py:246, 252`` ride in the norms, and the final norm rides in the
lm_head.  At decode sizes each norm/gate is applied by the GEMV kernel while it
stages its input rows, so there are no separate elementwise launches.  The same
trunk is what the executor captures in a HIP graph for one decode step.

Two keyword-only extensions select the embedding and lm_head formats of a
measured workload without changing the reference defaults: ``embedding``
(``"auto"``: the reference's choice, ``QuantizedParallelEmbedding`` when
``use_quantized`` else the dim-sharded ``ParallelEmbedding``; ``"vocab"``: the
vocab-sharded bf16 ``VocabParallelEmbedding``) and ``quantized_lm_head`` (a
quantized column-parallel lm_head in place of the dense one of ``:466-475``).
``forward(..., last_only=True)`` computes logits for the last position only,
the one ``generate`` reads (``worker/executor.py:267-270``).
"""
import logging
from typing import List, Optional, Tuple

import torch

from .. import _lib
from ..communicator import IdentityCommunicator
from ..kv_cache import KVCache, LayerKV, round_capacity
from .attention import ParallelAttention
from .column_linear import ColumnParallelLinear
from .embedding import ParallelEmbedding, QuantizedParallelEmbedding, VocabParallelEmbedding
from .mlp import ParallelMLP
from .quantized_linear import QuantizedColumnParallelLinear, QuantizedRowParallelLinear
from ._tensors import default_device, to_device

logger = logging.getLogger(__name__)


def run_sync(coro):
    """Drive a coroutine whose awaits complete immediately (identity collectives)."""
    try:
        coro.send(None)
    except StopIteration as stop:
        return stop.value
    coro.close()
    raise RuntimeError("a collective suspended: run the model under an event loop with await")


class RMSNorm:
    def __init__(self, hidden_size: int, eps: float = 1e-6, device=None):
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight: Optional[torch.Tensor] = None
        self.bias: Optional[torch.Tensor] = None
        self._device = device

    @property
    def device(self):
        if self._device is None:
            self._device = default_device()
        return self._device

    def load_weights(self, weight, bias=None):
        if tuple(weight.shape) != (self.hidden_size,):
            raise ValueError(f"Expected weight shape ({self.hidden_size},), got {tuple(weight.shape)}")
        self.weight = to_device(weight, self.device, torch.bfloat16)
        if bias is not None:
            if tuple(bias.shape) != (self.hidden_size,):
                raise ValueError(f"Expected bias shape ({self.hidden_size},), got {tuple(bias.shape)}")
            self.bias = to_device(bias, self.device, torch.bfloat16)

    def _check(self):
        if self.weight is None:
            raise RuntimeError("Weights not loaded")

    @property
    def fusable(self) -> bool:
        """Whether the projections that read this norm may normalise inside their own
        kernel (they take no LayerNorm-style bias; with one the norm runs on its own)."""
        return self.bias is None

    def __call__(self, x, residual=None, h_out=None, out=None):
        """``(x / sqrt(mean(x^2) + eps)) * weight``, then ``+ bias`` when one is loaded
        (LayerNorm-style, ``transformer.py:57-59``: the bias is added to the rounded
        normalised row and rounded again); with ``residual`` the input is
        ``x + residual`` (written to ``h_out`` when given)."""
        self._check()
        y = _lib.rms_norm(x, self.weight, self.eps, residual=residual, h_out=h_out, out=out)
        if self.bias is not None:
            y = _lib.add_row_bias(y, self.bias, out=y)
        return y


class ParallelTransformerBlock:
    def __init__(self, layer_idx: int, hidden_size: int, num_heads: int, intermediate_size: int, world_size: int,
                 rank: int, communicator=None, num_kv_heads: Optional[int] = None, rms_norm_eps: float = 1e-5,
                 attention_bias: bool = False, mlp_bias: bool = False, max_position_embeddings: int = 2048,
                 rope_base: float = 10000.0, mlp_activation: str = "silu", use_gated_mlp: bool = True,
                 use_quantized: bool = False, quantization_bits: int = 4, quantization_group_size: int = 64,
                 device=None):
        self.layer_idx = layer_idx
        self.hidden_size = hidden_size
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        self.input_layernorm = RMSNorm(hidden_size, eps=rms_norm_eps, device=device)
        self.post_attention_layernorm = RMSNorm(hidden_size, eps=rms_norm_eps, device=device)
        self.attention = ParallelAttention(hidden_size=hidden_size, num_heads=num_heads, world_size=world_size,
                                           rank=rank, communicator=communicator, num_kv_heads=num_kv_heads,
                                           bias=attention_bias, max_position_embeddings=max_position_embeddings,
                                           rope_base=rope_base, use_quantized=use_quantized,
                                           quantization_bits=quantization_bits,
                                           quantization_group_size=quantization_group_size, device=device)
        self.mlp = ParallelMLP(hidden_size=hidden_size, intermediate_size=intermediate_size, world_size=world_size,
                               rank=rank, communicator=communicator, activation=mlp_activation, bias=mlp_bias,
                               use_gated=use_gated_mlp, use_quantized=use_quantized,
                               quantization_bits=quantization_bits, quantization_group_size=quantization_group_size,
                               device=device)

    def load_weights(self, input_ln_weight, post_attn_ln_weight, attn_weights, mlp_weights):
        self.input_layernorm.load_weights(input_ln_weight)
        self.post_attention_layernorm.load_weights(post_attn_ln_weight)
        self.attention.load_shards(q_weight=attn_weights["q_weight"], q_bias=attn_weights.get("q_bias"),
                                   k_weight=attn_weights["k_weight"], k_bias=attn_weights.get("k_bias"),
                                   v_weight=attn_weights["v_weight"], v_bias=attn_weights.get("v_bias"),
                                   o_weight=attn_weights["o_weight"], o_bias=attn_weights.get("o_bias"))
        self.mlp.load_shards(up_weight=mlp_weights["up_weight"], up_bias=mlp_weights.get("up_bias"),
                             down_weight=mlp_weights["down_weight"], down_bias=mlp_weights.get("down_bias"),
                             gate_weight=mlp_weights.get("gate_weight"), gate_bias=mlp_weights.get("gate_bias"))

    async def forward(self, hidden_states, attention_mask=None, past_key_value=None, use_cache: bool = False):
        """Pre-norm residual block (``transformer.py:214-254``)."""
        xn = self.input_layernorm(hidden_states)
        attn_output, cache = await self.attention.forward(xn, attention_mask=attention_mask,
                                                          past_key_value=past_key_value, use_cache=use_cache)
        h = torch.empty_like(hidden_states)
        xn = self.post_attention_layernorm(hidden_states.contiguous(), residual=attn_output.contiguous(), h_out=h)
        mlp_output = await self.mlp.forward(xn)
        return _lib.add(h, mlp_output.contiguous()), cache

    @property
    def num_parameters(self) -> int:
        return (self.attention.num_parameters + self.mlp.num_parameters
                + 2 * self.hidden_size)


class StepBuffers:
    """Preallocated activations of one model step with B*S rows (decode: S = 1)."""

    def __init__(self, model: "ParallelTransformer", B: int, S: int, capacity: int):
        dev = model.device
        rows = B * S
        att = model.layers[0].attention
        mlp = model.layers[0].mlp
        bf = torch.bfloat16
        self.B, self.S = B, S
        self.ids = torch.zeros((B, S), dtype=torch.int32, device=dev)
        self.h = torch.empty((rows, model.hidden_size), dtype=bf, device=dev)
        self.h2 = torch.empty_like(self.h)
        self.xn = torch.empty_like(self.h)
        self.qkv = torch.empty((rows, att.qkv_width), dtype=bf, device=dev)
        self.attn = torch.empty((rows, att.local_hidden), dtype=bf, device=dev)
        self.gu = torch.empty((rows, 2 * mlp.local_intermediate), dtype=bf, device=dev)
        self.act = torch.empty((rows, mlp.local_intermediate), dtype=bf, device=dev)
        self.hn = torch.empty((B, model.hidden_size), dtype=bf, device=dev)
        H, Hk, D, T_cap = att.local_num_heads, att.local_num_kv_heads, att.head_dim, round_capacity(capacity)
        ws = _lib.attention_workspace_bytes(B, S, H, Hk, D, T_cap)
        if S == 1:
            ws = max(ws, _lib.attention_decode_workspace_bytes(B, H, Hk, D, T_cap))
        self.workspace = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        # greedy-head workspace: zero, and every decode_head call leaves it zero
        self.head_ws = torch.zeros(_lib.DECODE_HEAD_WORKSPACE_BYTES // 4, dtype=torch.int32, device=dev)
        self.plan = None          # a TrunkPlan when the whole trunk runs as one launch


class ParallelTransformer:
    def __init__(self, vocab_size: int, hidden_size: int, num_layers: int, num_heads: int, intermediate_size: int,
                 world_size: int, rank: int, communicator=None, num_kv_heads: Optional[int] = None,
                 max_position_embeddings: int = 2048, rms_norm_eps: float = 1e-5, tie_word_embeddings: bool = False,
                 rope_base: float = 10000.0, mlp_activation: str = "silu", use_gated_mlp: bool = True,
                 use_quantized: bool = False, quantization_bits: int = 4, quantization_group_size: int = 64, *,
                 embedding: str = "auto", quantized_lm_head: bool = False, device=None):
        if communicator is None and world_size == 1:
            communicator = IdentityCommunicator()
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads if num_kv_heads else num_heads
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        self.tie_word_embeddings = tie_word_embeddings
        self.use_quantized = use_quantized
        self.quantization_bits = quantization_bits
        self.quantization_group_size = quantization_group_size
        self.max_position_embeddings = max_position_embeddings
        self._device = device
        if embedding == "auto":
            embedding = "quantized" if use_quantized else "dense"
        if embedding == "quantized":
            self.embed_tokens = QuantizedParallelEmbedding(vocab_size=vocab_size, embedding_dim=hidden_size,
                                                           world_size=world_size, rank=rank,
                                                           communicator=communicator,
                                                           group_size=quantization_group_size,
                                                           bits=quantization_bits, device=device)
        elif embedding == "dense":
            self.embed_tokens = ParallelEmbedding(vocab_size=vocab_size, embedding_dim=hidden_size,
                                                  world_size=world_size, rank=rank, gather_output=True,
                                                  communicator=communicator, device=device)
        elif embedding == "vocab":
            self.embed_tokens = VocabParallelEmbedding(vocab_size=vocab_size, embedding_dim=hidden_size,
                                                       world_size=world_size, rank=rank, communicator=communicator,
                                                       device=device)
        else:
            raise ValueError(f"unknown embedding kind {embedding!r}")
        self.embedding_kind = embedding
        self.layers: List[ParallelTransformerBlock] = [
            ParallelTransformerBlock(layer_idx=i, hidden_size=hidden_size, num_heads=num_heads,
                                     intermediate_size=intermediate_size, world_size=world_size, rank=rank,
                                     communicator=communicator, num_kv_heads=num_kv_heads,
                                     rms_norm_eps=rms_norm_eps, max_position_embeddings=max_position_embeddings,
                                     rope_base=rope_base, mlp_activation=mlp_activation,
                                     use_gated_mlp=use_gated_mlp, use_quantized=use_quantized,
                                     quantization_bits=quantization_bits,
                                     quantization_group_size=quantization_group_size, device=device)
            for i in range(num_layers)]
        self.norm = RMSNorm(hidden_size, eps=rms_norm_eps, device=device)
        if tie_word_embeddings:
            self.lm_head = None
        elif quantized_lm_head:
            self.lm_head = QuantizedColumnParallelLinear(hidden_size, vocab_size, world_size, rank, bias=False,
                                                         gather_output=True, communicator=communicator,
                                                         bits=quantization_bits,
                                                         group_size=quantization_group_size, device=device)
        else:
            self.lm_head = ColumnParallelLinear(hidden_size, vocab_size, world_size, rank, bias=False,
                                                gather_output=True, communicator=communicator, device=device)

    @property
    def device(self):
        if self._device is None:
            self._device = default_device()
        return self._device

    # ---------------------------------------------------------------- loading

    def load_embedding_weights(self, weight):
        self.embed_tokens.load_shard_direct(weight)

    def load_quantized_embedding_weights(self, weight, scales, biases):
        if not isinstance(self.embed_tokens, QuantizedParallelEmbedding):
            raise RuntimeError("Cannot load quantized embeddings into non-quantized model")
        self.embed_tokens.load_quantized_shard(weight, scales, biases)

    def load_lm_head_weights(self, weight):
        if self.lm_head is not None:
            self.lm_head.load_shard_direct(weight)

    def load_quantized_lm_head_weights(self, weight, scales, biases):
        if not isinstance(self.lm_head, QuantizedColumnParallelLinear):
            raise RuntimeError("the lm_head is not quantized (construct with quantized_lm_head=True)")
        self.lm_head.load_quantized_shard(weight, scales, biases)

    def load_norm_weights(self, weight):
        self.norm.load_weights(weight)

    # ---------------------------------------------------------------- compute

    def new_cache(self, batch: int, capacity: int) -> KVCache:
        att = self.layers[0].attention
        return KVCache(self.num_layers, batch, att.local_num_kv_heads, att.head_dim, capacity, device=self.device)

    def _embed_sync(self, input_ids, out=None):
        if isinstance(self.embed_tokens, VocabParallelEmbedding):
            return self.embed_tokens.forward_sync(input_ids, out=out)
        emb = self.embed_tokens.forward_sync(input_ids)
        if out is not None:
            out.copy_(emb.reshape(out.shape))
            return out
        return emb

    async def _embed(self, input_ids, out=None):
        emb = self._embed_sync(input_ids, out=out)
        if self.world_size > 1 and self.communicator is not None:
            if isinstance(self.embed_tokens, ParallelEmbedding):
                emb = await self.communicator.all_gather(emb, dim=-1)
            else:
                emb = await self.communicator.all_reduce(emb, op="sum")
        return emb

    async def _trunk(self, h, cache: KVCache, B: int, S: int, bufs: Optional[StepBuffers] = None, mask=None):
        """Residual stream ``h [B*S, hidden]`` through every layer (``mask``: the
        additive attention mask every layer's attention adds to its scores).

        Each RMSNorm (with the residual add before it) runs inside the projection
        that reads it, or, above 8 rows, inside the projection that feeds the
        residual add (o_proj and down_proj, their split-K pass folded into the
        norm's), and the SiLU gate inside the gate|up product.  The residual stream
        alternates between two buffers (a kernel's h_out may not alias its input).
        Returns (h, the last layer's MLP output whose residual add is pending)."""
        h_alt = bufs.h2 if bufs is not None else torch.empty_like(h)
        xn_buf = bufs.xn if bufs is not None else None
        pending = None
        xn_next = None          # the next layer's normalised input, when down_proj computed it
        L = len(self.layers)
        for i, layer in enumerate(self.layers):
            att, mlp = layer.attention, layer.mlp
            if xn_next is not None:
                qkv = att.qkv(xn_next, out=bufs.qkv if bufs is not None else None)
            else:
                qkv, _ = att.qkv.norm_call(h, layer.input_layernorm, residual=pending,
                                           h_out=h_alt if pending is not None else None, xn_out=xn_buf,
                                           out=bufs.qkv if bufs is not None else None)
                if pending is not None:
                    h, h_alt = h_alt, h
            a = att.attend_qkv(qkv, B, S, cache[i], out=bufs.attn if bufs else None,
                               workspace=bufs.workspace if bufs else None, mask=mask)
            act_out = bufs.act if bufs is not None else None
            gu_out = bufs.gu if bufs is not None else None
            if self._folds(att.o_proj, layer.post_attention_layernorm, B * S):
                # o_proj, the residual add and the post-attention norm in one call: its
                # split-K pass runs inside the norm's
                _, xn = att.o_proj.forward_add_norm(a, h, layer.post_attention_layernorm, h_out=h_alt, xn_out=xn_buf)
                act = mlp.act_from_xn(xn, act_out=act_out, gu_out=gu_out)
            else:
                o = await att.o_proj.forward(a)
                act = mlp.act_call(h, layer.post_attention_layernorm, residual=o, h_out=h_alt, xn_out=xn_buf,
                                   act_out=act_out, gu_out=gu_out)
            h, h_alt = h_alt, h
            xn_next = None
            if i + 1 < L and self._folds(mlp.down_proj, self.layers[i + 1].input_layernorm, B * S):
                # down_proj, the residual add and the next layer's input norm in one call
                h_new, xn_next = mlp.down_proj.forward_add_norm(act, h, self.layers[i + 1].input_layernorm,
                                                                h_out=h_alt, xn_out=xn_buf)
                h, h_alt = h_new, h
                pending = None
            else:
                pending = await mlp.down_proj.forward(act)
        return h, pending

    @staticmethod
    def _folds(proj, norm, rows: int) -> bool:
        """Whether a row-parallel projection runs with its residual add and the next
        norm folded in (sc_qmm_add_rmsnorm_bf16): a quantized projection with an
        identity all-reduce, a bias-free norm, and more than 8 rows (up to 8 the
        decode GEMV applies the norm while staging the next product's input, which
        is one launch fewer still)."""
        return (rows > 8 and isinstance(proj, QuantizedRowParallelLinear) and proj.folds_norm and norm.fusable)

    async def _head(self, h, pending, B, S, last_only, hn_out=None):
        """Final RMSNorm (of h + pending, when a residual add is pending) and lm_head."""
        if last_only and S > 1:
            h = h.reshape(B, S, -1)[:, -1].contiguous()
            if pending is not None:
                pending = pending.reshape(B, S, -1)[:, -1].contiguous()
        lm = self.lm_head
        if isinstance(lm, QuantizedColumnParallelLinear) and self.norm.fusable:
            if lm.quantized_weight is None:
                raise RuntimeError("Weight not loaded")
            self.norm._check()
            # the final norm runs inside the lm_head kernel
            logits, _ = _lib.qmm_rmsnorm(h, self.norm.weight, self.norm.eps, lm.quantized_weight, lm.scales,
                                         lm.biases_quant, residual=pending, xn_out=hn_out,
                                         bias=lm.bias if lm.has_bias else None, bits=lm.bits,
                                         group_size=lm.group_size)
            if lm.gather_output:
                if self.communicator is None:
                    raise RuntimeError("Communicator required for gather_output=True")
                logits = await self.communicator.all_gather(logits, dim=-1)
            return logits
        hn = self.norm(h, residual=pending, h_out=None, out=hn_out)
        if self.tie_word_embeddings:
            emb = self.embed_tokens
            w = emb.dequantize_weight() if hasattr(emb, "dequantize_weight") else emb.weight
            logits = hn @ w.T
            if self.communicator is not None:
                logits = await self.communicator.all_gather(logits, dim=-1)
        else:
            logits = await lm.forward(hn)
        return logits

    async def forward(self, input_ids, attention_mask=None, past_key_values=None, use_cache: bool = False, *,
                      last_only: bool = False):
        """Logits ``[batch, seq (or 1), vocab]`` and the cache (``transformer.py:516-577``).

        ``past_key_values``: a :class:`KVCache` (appended in place, returned as is),
        a list of reference-layout ``(k, v)`` tuples (the grown list is returned),
        or ``None``.  ``attention_mask``: an additive mask broadcastable to
        ``[batch, local heads, seq, cached + seq keys]``, passed to every layer
        (``transformer.py:548-553``)."""
        ids = input_ids if isinstance(input_ids, torch.Tensor) else torch.as_tensor(input_ids)
        ids = ids.to(self.device)
        if ids.dim() != 2:
            raise ValueError("input_ids must be [batch, seq_len]")
        B, S = ids.shape
        if isinstance(past_key_values, KVCache):
            cache, tuples = past_key_values, False
        else:
            T0 = 0 if not past_key_values else past_key_values[0][0].shape[2]
            cache, tuples = self.new_cache(B, T0 + S), True
            if past_key_values:
                cache.load_tuples(past_key_values)
        cache.check_room(S)
        h = (await self._embed(ids)).reshape(B * S, self.hidden_size).contiguous()
        h, pending = await self._trunk(h, cache, B, S, mask=attention_mask)
        logits = await self._head(h, pending, B, S, last_only)
        cache.advance(S)
        new_cache = (cache.as_tuples() if tuples else cache) if use_cache else None
        return logits.reshape(B, 1 if (last_only and S > 1) else S, -1), new_cache

    def decode_step(self, bufs: StepBuffers, cache: KVCache, tokens: torch.Tensor, logits_out=None):
        """One greedy decode step on device, no host synchronisation: embed
        ``bufs.ids``, run every layer (appending at ``cache.counters[0]``), argmax the
        logits into ``bufs.ids`` and ``tokens[:, step]``, then advance the cache
        length and the step counter.  Captured once, replayed per token."""
        B = bufs.B
        if bufs.plan is not None:
            # embedding and every layer in one persistent launch (batch 1)
            h, pending = bufs.plan.run().view(B, self.hidden_size), None
        else:
            h = self._embed_sync(bufs.ids, out=bufs.h.view(B, 1, self.hidden_size)).view(B, self.hidden_size)
            h, pending = run_sync(self._trunk(h, cache, B, 1, bufs))
        lm = self.lm_head
        if (isinstance(lm, QuantizedColumnParallelLinear) and (not lm.gather_output or self.world_size == 1)
                and self.norm.fusable):
            # final norm, lm_head, greedy selection and counter advance in one call
            # (at batch 1 the lm_head GEMV selects the token while writing the logits)
            if lm.quantized_weight is None:
                raise RuntimeError("Weight not loaded")
            self.norm._check()
            logits, _ = _lib.decode_head(h, self.norm.weight, self.norm.eps, lm.quantized_weight, lm.scales,
                                         lm.biases_quant, bufs.ids.view(-1), bufs.head_ws, residual=pending,
                                         xn_out=bufs.hn, bias=lm.bias if lm.has_bias else None, bits=lm.bits,
                                         group_size=lm.group_size, tokens=tokens, step=cache.counters[1:],
                                         counters=cache.counters, n_counters=2)
            return logits
        logits = run_sync(self._head(h, pending, B, 1, True, hn_out=bufs.hn))
        _lib.argmax(logits.reshape(B, -1), ids=bufs.ids.view(-1), tokens=tokens, step=cache.counters[1:])
        _lib.add_i32(cache.counters, 1, n=2)
        return logits

    @property
    def num_parameters(self) -> int:
        n = sum(layer.num_parameters for layer in self.layers) + self.embed_tokens.num_parameters
        if self.lm_head is not None:
            n += self.lm_head.num_parameters
        return n + self.hidden_size

    def get_layer(self, idx: int) -> ParallelTransformerBlock:
        if idx < 0 or idx >= len(self.layers):
            raise IndexError(f"Layer index {idx} out of range [0, {len(self.layers)})")
        return self.layers[idx]
