"""Tensor-parallel attention over the HIP kernels (one rank's heads).

Drop-in for ``src/shardcompute/parallel/attention.py``: ``RoPE`` (``:19-151``)
and ``ParallelAttention`` (``:154-622``) keep their constructor arguments,
attributes, loaders and forward signatures.  Per call:

1. one fused q|k|v quantized GEMV/GEMM (``sc_qmm_bf16``; the three projections
   of ``:406-408`` stacked, bit-identical per column),
2. ``sc_rope_append_kv_bf16``: rotate-half RoPE on q and k with fp32 cos/sin
   tables, k and v appended to the preallocated cache (``:421-435``),
3. ``sc_attention_bf16``: causal GQA softmax attention on MFMA (``:437-466``),
4. the row-parallel o_proj (``sc_qmm_bf16``), all-reduce = identity at world_size 1.

``past_key_value`` may be a :class:`~shardcompute_amd.kv_cache.LayerKV` (the
preallocated cache; appended in place and returned), a reference-layout tuple
``(k, v)`` of ``[batch, kv_heads, T, head_dim]`` (copied into a temporary cache;
the grown tuple is returned, as the reference does), or ``None``.  With a
``LayerKV`` the owner of the cache advances its length once per model step
(every layer appends at the same positions).
"""
import logging
import math
from typing import Optional, Tuple

import numpy as np
import torch

from .. import _lib
from ..kv_cache import KVCache, LayerKV, round_capacity
from ._fused import FusedColumns
from .column_linear import ColumnParallelLinear
from .quantized_linear import QuantizedColumnParallelLinear, QuantizedRowParallelLinear
from .row_linear import RowParallelLinear

logger = logging.getLogger(__name__)


def rope_tables_np(head_dim: int, base: float, scaling_factor: float, length: int):
    """fp32 cos/sin ``[length, head_dim/2]`` as ``RoPE._update_cache`` builds them
    (``attention.py:54-59, 66-92``): ``inv_freq = 1 / base^(2i/d)``,
    positions ``t (/ scaling_factor)``, ``freqs = outer(t, inv_freq)``."""
    inv_freq = (np.float32(1.0) / (np.float32(base) ** (np.arange(0, head_dim, 2, dtype=np.float32)
                                                          / np.float32(head_dim)))).astype(np.float32)
    t = np.arange(length, dtype=np.float32)
    if scaling_factor != 1.0:
        t = (t / np.float32(scaling_factor)).astype(np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


class RoPE:
    """Rotary embeddings (``attention.py:19-151``) with device-resident fp32 tables."""

    def __init__(self, head_dim: int, max_position_embeddings: int = 2048, base: float = 10000.0,
                 scaling_factor: float = 1.0):
        self.head_dim = head_dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base
        self.scaling_factor = scaling_factor
        self.inv_freq = (1.0 / (np.float32(base) ** (np.arange(0, head_dim, 2, dtype=np.float32)
                                                      / np.float32(head_dim)))).astype(np.float32)
        self._tables = {}

    def tables(self, length: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
        """(cos, sin) fp32 ``[>= length, head_dim/2]`` on ``device`` (grown by doubling, min 256)."""
        key = str(device)
        cur = self._tables.get(key)
        if cur is None or cur[0].shape[0] < length:
            have = 0 if cur is None else cur[0].shape[0]
            n = max(int(length), 2 * have, 256, self.max_position_embeddings)
            c, s = rope_tables_np(self.head_dim, self.base, self.scaling_factor, n)
            cur = (torch.from_numpy(c).to(device), torch.from_numpy(s).to(device))
            self._tables[key] = cur
        return cur

    def __call__(self, q: torch.Tensor, k: torch.Tensor, position_offset: int = 0):
        """Rotate q ``[B, H, S, D]`` and k ``[B, Hkv, S, D]`` for positions offset..offset+S-1."""
        B, H, S, D = q.shape
        Hkv = k.shape[1]
        rows = torch.zeros((B * S, (H + 2 * Hkv) * D), dtype=torch.bfloat16, device=q.device)
        rows[:, :H * D] = q.transpose(1, 2).reshape(B * S, H * D)
        rows[:, H * D:(H + Hkv) * D] = k.transpose(1, 2).reshape(B * S, Hkv * D)
        cache = KVCache(1, B, Hkv, D, S, device=q.device)
        cos_t, sin_t = self.tables(position_offset + S, q.device)
        _lib.rope_append_kv(rows, B, S, H, Hkv, D, cos_t, sin_t, cache.k[0], cache.vt[0], cache.counters,
                            pos_offset=position_offset)
        q_rot = rows[:, :H * D].reshape(B, S, H, D).transpose(1, 2).contiguous()
        k_rot = cache.k[0][:, :, :S].contiguous()
        return q_rot, k_rot


class ParallelAttention:
    def __init__(self, hidden_size: int, num_heads: int, world_size: int, rank: int, communicator=None,
                 num_kv_heads: Optional[int] = None, head_dim: Optional[int] = None, bias: bool = False,
                 attention_dropout: float = 0.0, max_position_embeddings: int = 2048, rope_base: float = 10000.0,
                 rope_scaling_factor: float = 1.0, use_quantized: bool = False, quantization_bits: int = 4,
                 quantization_group_size: int = 64, device=None):
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        if num_heads % world_size != 0:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by world_size ({world_size})")
        self.local_num_heads = num_heads // world_size
        self.head_dim = head_dim if head_dim else hidden_size // num_heads
        self.local_hidden = self.local_num_heads * self.head_dim
        self.num_kv_heads = num_kv_heads if num_kv_heads else num_heads
        if self.num_kv_heads % world_size != 0:
            raise ValueError(f"num_kv_heads ({self.num_kv_heads}) must be divisible by world_size")
        self.local_num_kv_heads = self.num_kv_heads // world_size
        self.local_kv_hidden = self.local_num_kv_heads * self.head_dim
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self.rope = RoPE(head_dim=self.head_dim, max_position_embeddings=max_position_embeddings, base=rope_base,
                         scaling_factor=rope_scaling_factor)
        self.use_quantized = use_quantized
        D, H, Hk = self.head_dim, num_heads, self.num_kv_heads
        if use_quantized:
            def col(out):
                return QuantizedColumnParallelLinear(hidden_size, out, world_size, rank, bias=bias,
                                                     gather_output=False, bits=quantization_bits,
                                                     group_size=quantization_group_size, device=device)
            self.q_proj, self.k_proj, self.v_proj = col(H * D), col(Hk * D), col(Hk * D)
            self.o_proj = QuantizedRowParallelLinear(H * D, hidden_size, world_size, rank, bias=bias,
                                                     input_is_partitioned=True, communicator=communicator,
                                                     bits=quantization_bits, group_size=quantization_group_size,
                                                     device=device)
        else:
            def col(out):
                return ColumnParallelLinear(hidden_size, out, world_size, rank, bias=bias, gather_output=False,
                                            device=device)
            self.q_proj, self.k_proj, self.v_proj = col(H * D), col(Hk * D), col(Hk * D)
            self.o_proj = RowParallelLinear(H * D, hidden_size, world_size, rank, bias=bias,
                                            input_is_partitioned=True, communicator=communicator, device=device)
        self.qkv = FusedColumns([self.q_proj, self.k_proj, self.v_proj])

    # ---------------------------------------------------------------- loading

    def load_shards(self, q_weight, q_bias, k_weight, k_bias, v_weight, v_bias, o_weight, o_bias):
        self.q_proj.load_shard_direct(q_weight, q_bias)
        self.k_proj.load_shard_direct(k_weight, k_bias)
        self.v_proj.load_shard_direct(v_weight, v_bias)
        self.o_proj.load_shard_direct(o_weight, o_bias)

    def load_quantized_shards(self, q_weight, q_scales, q_biases, q_linear_bias, k_weight, k_scales, k_biases,
                              k_linear_bias, v_weight, v_scales, v_biases, v_linear_bias, o_weight, o_scales,
                              o_biases, o_linear_bias):
        if not self.use_quantized:
            raise RuntimeError("Cannot load quantized shards into non-quantized attention")
        self.q_proj.load_quantized_shard(q_weight, q_scales, q_biases, q_linear_bias)
        self.k_proj.load_quantized_shard(k_weight, k_scales, k_biases, k_linear_bias)
        self.v_proj.load_quantized_shard(v_weight, v_scales, v_biases, v_linear_bias)
        self.o_proj.load_quantized_shard(o_weight, o_scales, o_biases, o_linear_bias)

    # ---------------------------------------------------------------- compute

    @property
    def qkv_width(self):
        return (self.local_num_heads + 2 * self.local_num_kv_heads) * self.head_dim

    def attend(self, x2, B, S, kv: LayerKV, out=None, qkv_out=None, workspace=None, pos_offset=0, mask=None):
        """Core of the forward: x2 ``[B*S, hidden]`` -> attention output ``[B*S, local_hidden]``
        (before o_proj), appending the S new positions at ``kv.counters[0]``."""
        return self.attend_qkv(self.qkv(x2, out=qkv_out), B, S, kv, out=out, workspace=workspace,
                               pos_offset=pos_offset, mask=mask)

    def attend_qkv(self, qkv, B, S, kv: LayerKV, out=None, workspace=None, pos_offset=0, mask=None):
        """RoPE, cache append and attention on an already computed q|k|v product.

        One position per sequence (decode) runs as the fused decode attention
        (RoPE, append and attention in one launch, plus the range merge), with the
        mask when one is given.  ``mask``
        is the reference's additive ``attention_mask``, broadcastable to
        ``[B, local heads, S, cached + S keys]`` (``attention.py:449-450``)."""
        H, Hk, D = self.local_num_heads, self.local_num_kv_heads, self.head_dim
        cos_t, sin_t = self.rope.tables(kv.cache.capacity + pos_offset, qkv.device)
        n_keys = kv.length + S
        if S == 1 and H // Hk <= 16:
            return _lib.attention_decode(qkv, B, H, Hk, D, cos_t, sin_t, kv.k, kv.vt, kv.counters, self.scale,
                                         pos_offset=pos_offset, out=out, workspace=workspace, mask=mask,
                                         n_keys=n_keys if mask is not None else None)
        _lib.rope_append_kv(qkv, B, S, H, Hk, D, cos_t, sin_t, kv.k, kv.vt, kv.counters, pos_offset=pos_offset)
        return _lib.attention(qkv, B, S, H, Hk, D, kv.k, kv.vt, kv.counters, self.scale, out=out,
                              workspace=workspace, mask=mask, n_keys=n_keys)

    def _prepare_cache(self, past_key_value, B, S, device):
        """-> (LayerKV, temp cache or None, whether to return a tuple)."""
        if isinstance(past_key_value, LayerKV):
            past_key_value.cache.check_room(S)
            return past_key_value, None
        T0 = 0 if past_key_value is None else past_key_value[0].shape[2]
        tmp = KVCache(1, B, self.local_num_kv_heads, self.head_dim, round_capacity(T0 + S), device=device)
        if past_key_value is not None:
            tmp.load_tuples([past_key_value])
        return tmp[0], tmp

    def _attn_core(self, hidden_states, attention_mask, past_key_value, use_cache):
        B, S, _ = hidden_states.shape
        x2 = hidden_states.reshape(B * S, -1)
        kv, tmp = self._prepare_cache(past_key_value, B, S, hidden_states.device)
        a = self.attend(x2, B, S, kv, mask=attention_mask)
        if tmp is not None:
            tmp.advance(S)
            new_cache = tmp[0].as_tuple() if use_cache else None
        else:
            new_cache = kv if use_cache else None
        return a.reshape(B, S, self.local_hidden), new_cache

    async def forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None,
                      past_key_value=None, use_cache: bool = False):
        a, new_cache = self._attn_core(hidden_states, attention_mask, past_key_value, use_cache)
        output = await self.o_proj.forward(a)
        return output, new_cache

    def forward_sync_partial(self, hidden_states: torch.Tensor, attention_mask=None, position_offset: int = 0):
        """Attention without all-reduce and without cache (``attention.py:473-520``):
        the S positions attend causally among themselves, rotated for
        ``position_offset + s``; ``attention_mask`` is added to the scaled scores
        (``attention.py:507-508``)."""
        B, S, _ = hidden_states.shape
        tmp = KVCache(1, B, self.local_num_kv_heads, self.head_dim, S, device=hidden_states.device)
        a = self.attend(hidden_states.reshape(B * S, -1), B, S, tmp[0], pos_offset=position_offset,
                        mask=attention_mask)
        return self.o_proj.forward_partial(a.reshape(B, S, self.local_hidden))

    def forward_partial_with_cache(self, hidden_states: torch.Tensor, attention_mask=None, past_key_value=None,
                                   use_cache: bool = False):
        a, new_cache = self._attn_core(hidden_states, attention_mask, past_key_value, use_cache)
        return self.o_proj.forward_partial(a), new_cache

    @property
    def num_parameters(self) -> int:
        return (self.q_proj.num_parameters + self.k_proj.num_parameters + self.v_proj.num_parameters
                + self.o_proj.num_parameters)
