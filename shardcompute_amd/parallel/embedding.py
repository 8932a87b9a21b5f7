"""Embedding layers over the HIP masked-gather kernels.

Drop-in for ``src/shardcompute/parallel/embedding.py``:

* ``ParallelEmbedding`` (``:12-188``): table sharded along the embedding dim;
  lookup = ``sc_vocab_gather_bf16`` over the whole vocabulary.
* ``QuantizedParallelEmbedding`` (``:191-394``): vocab-sharded quantized table;
  lookup = ``sc_qembed_gather_bf16`` (offset, range mask, clip, take,
  dequantize, zero out-of-shard rows in one kernel).
* ``VocabParallelEmbedding`` (a stub in the reference, ``:397-418``): the same
  vocab-sharded mask semantics on a bf16 table, bit-exact, via
  ``sc_vocab_gather_bf16``.  It keeps the stub's constructor signature.
"""
import logging
from typing import Optional

import torch

from .. import _lib
from ._tensors import default_device, packed, to_device

logger = logging.getLogger(__name__)


class _DeviceMixin:
    @property
    def device(self):
        if self._device is None:
            self._device = default_device()
        return self._device


class ParallelEmbedding(_DeviceMixin):
    """Embedding split by embedding dimension (``embedding.py:12-188``)."""

    def __init__(self, vocab_size: int, embedding_dim: int, world_size: int, rank: int, gather_output: bool = True,
                 communicator=None, padding_idx: Optional[int] = None, device=None):
        self.vocab_size = vocab_size
        self.embedding_dim = embedding_dim
        self.world_size = world_size
        self.rank = rank
        self.gather_output = gather_output
        self.communicator = communicator
        self.padding_idx = padding_idx
        if embedding_dim % world_size != 0:
            raise ValueError(f"embedding_dim ({embedding_dim}) must be divisible by world_size ({world_size})")
        self.local_embedding_dim = embedding_dim // world_size
        self.col_start = rank * self.local_embedding_dim
        self.col_end = self.col_start + self.local_embedding_dim
        self.weight: Optional[torch.Tensor] = None
        self._device = device

    def load_shard(self, full_weight):
        w = to_device(full_weight, self.device, torch.bfloat16)
        self.weight = w[:, self.col_start:self.col_end].contiguous()

    def load_shard_direct(self, weight_shard):
        if weight_shard is None:
            logger.warning("load_shard_direct called with None weight, skipping")
            return
        expected = (self.vocab_size, self.local_embedding_dim)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}")
        self.weight = to_device(weight_shard, self.device, torch.bfloat16)

    def _lookup(self, input_ids):
        if self.weight is None:
            raise RuntimeError("Embedding weights not loaded")
        emb = _lib.vocab_gather(input_ids.to(self.device), self.weight, 0)
        if self.padding_idx is not None:
            mask = (input_ids.to(self.device) == self.padding_idx)[..., None]
            emb = torch.where(mask, torch.zeros_like(emb), emb)
        return emb

    async def forward(self, input_ids):
        emb = self._lookup(input_ids)
        if self.gather_output:
            if self.communicator is None:
                raise RuntimeError("Communicator required for gather_output=True")
            emb = await self.communicator.all_gather(emb, dim=-1)
        return emb

    def forward_sync(self, input_ids):
        return self._lookup(input_ids)

    @property
    def num_parameters(self) -> int:
        return self.vocab_size * self.local_embedding_dim

    def __repr__(self):
        return (f"ParallelEmbedding(vocab_size={self.vocab_size}, embedding_dim={self.embedding_dim}, "
                f"local_embedding_dim={self.local_embedding_dim}, rank={self.rank}/{self.world_size})")


class _VocabShard:
    def _init_vocab(self, vocab_size, world_size, rank):
        if vocab_size % world_size != 0:
            raise ValueError(f"vocab_size ({vocab_size}) must be divisible by world_size ({world_size})")
        self.local_vocab_size = vocab_size // world_size
        self.vocab_start = rank * self.local_vocab_size
        self.vocab_end = self.vocab_start + self.local_vocab_size


class QuantizedParallelEmbedding(_DeviceMixin, _VocabShard):
    """Vocab-sharded quantized embedding (``embedding.py:191-394``)."""

    def __init__(self, vocab_size: int, embedding_dim: int, world_size: int, rank: int, communicator=None,
                 group_size: int = 64, bits: int = 4, device=None):
        self.vocab_size = vocab_size
        self.embedding_dim = embedding_dim
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        self.group_size = group_size
        self.bits = bits
        self._init_vocab(vocab_size, world_size, rank)
        self.quantized_weight: Optional[torch.Tensor] = None
        self.scales: Optional[torch.Tensor] = None
        self.biases_quant: Optional[torch.Tensor] = None
        self._device = device

    def load_quantized_shard(self, quantized_weight, scales, biases):
        self.quantized_weight = packed(quantized_weight, self.device)
        self.scales = to_device(scales, self.device, torch.bfloat16)
        self.biases_quant = to_device(biases, self.device, torch.bfloat16)

    def load_shard_direct(self, weight_shard):
        if weight_shard is None:
            logger.warning("load_shard_direct called with None weight, skipping")
            return
        expected = (self.local_vocab_size, self.embedding_dim)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}. "
                             f"For quantized embeddings, use load_quantized_shard() with weight, scales, and biases.")
        w = to_device(weight_shard, self.device, torch.float32)
        self.quantized_weight, self.scales, self.biases_quant = _lib.quantize(w, self.bits, self.group_size)

    def _lookup(self, input_ids):
        if self.quantized_weight is None:
            raise RuntimeError("Embedding weights not loaded")
        return _lib.qembed_gather(input_ids.to(self.device), self.quantized_weight, self.scales, self.biases_quant,
                                  self.vocab_start, self.bits, self.group_size)

    async def forward(self, input_ids):
        emb = self._lookup(input_ids)
        if self.communicator is not None:
            emb = await self.communicator.all_reduce(emb, op="sum")
        return emb

    def forward_sync(self, input_ids):
        return self._lookup(input_ids)

    @property
    def weight(self):
        return self.quantized_weight

    def dequantize_weight(self):
        if self.quantized_weight is None or self.scales is None or self.biases_quant is None:
            raise RuntimeError("Quantized embedding weights not loaded")
        return _lib.dequantize(self.quantized_weight, self.scales, self.biases_quant, self.bits, self.group_size)

    @property
    def num_parameters(self) -> int:
        return self.local_vocab_size * self.embedding_dim

    def __repr__(self):
        return (f"QuantizedParallelEmbedding(vocab_size={self.vocab_size}, local_vocab_size={self.local_vocab_size}, "
                f"embedding_dim={self.embedding_dim}, rank={self.rank}/{self.world_size}, bits={self.bits})")


class VocabParallelEmbedding(_DeviceMixin, _VocabShard):
    """Vocab-sharded bf16 embedding with the reference's mask semantics.

    Rank ``r`` owns rows ``[r * V / ws, (r + 1) * V / ws)``; ids outside that
    range produce +0.0 rows, in-range ids copy their row bit for bit
    (``embedding.py:322-356`` applied to a bf16 table).  ``forward`` sums the
    ranks' rows with the communicator's all-reduce when one is given.
    """

    def __init__(self, vocab_size: int, embedding_dim: int, world_size: int, rank: int, communicator=None,
                 device=None):
        self.vocab_size = vocab_size
        self.embedding_dim = embedding_dim
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        self._init_vocab(vocab_size, world_size, rank)
        self.weight: Optional[torch.Tensor] = None
        self._device = device

    def load_shard(self, full_weight):
        """Keep this rank's rows of the full ``[vocab_size, embedding_dim]`` table."""
        if tuple(full_weight.shape) != (self.vocab_size, self.embedding_dim):
            raise ValueError(f"Full weight shape {tuple(full_weight.shape)} doesn't match "
                             f"({self.vocab_size}, {self.embedding_dim})")
        self.weight = to_device(full_weight[self.vocab_start:self.vocab_end], self.device, torch.bfloat16)

    def load_shard_direct(self, weight_shard):
        if weight_shard is None:
            logger.warning("load_shard_direct called with None weight, skipping")
            return
        expected = (self.local_vocab_size, self.embedding_dim)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}")
        self.weight = to_device(weight_shard, self.device, torch.bfloat16)

    def forward_sync(self, input_ids, out=None):
        if self.weight is None:
            raise RuntimeError("Embedding weights not loaded")
        return _lib.vocab_gather(input_ids.to(self.device), self.weight, self.vocab_start, out=out)

    async def forward(self, input_ids):
        emb = self.forward_sync(input_ids)
        if self.communicator is not None:
            emb = await self.communicator.all_reduce(emb, op="sum")
        return emb

    @property
    def num_parameters(self) -> int:
        return self.local_vocab_size * self.embedding_dim

    def __repr__(self):
        return (f"VocabParallelEmbedding(vocab_size={self.vocab_size}, local_vocab_size={self.local_vocab_size}, "
                f"embedding_dim={self.embedding_dim}, rank={self.rank}/{self.world_size})")
