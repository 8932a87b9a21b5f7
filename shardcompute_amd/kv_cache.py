"""Preallocated per-layer KV cache on the GPU.

The reference grows its cache by concatenation: every step returns new
``(k, v)`` arrays ``[batch, kv_heads, seq, head_dim]`` per layer
(``parallel/attention.py:429-433``, ``worker/executor.py:134-136``).  Here the
cache is allocated once, for ``capacity`` positions, and the kernels append in
place:

* ``k``  ``[layers, batch, kv_heads, capacity, head_dim]`` bf16
* ``vt`` ``[layers, batch, kv_heads, head_dim, capacity]`` bf16 (values
  transposed, so the attention kernel reads keys-contiguous rows of V)
* ``counters`` int32 ``[2]`` on the device: ``[cached positions, decode step]``.
  Kernels read the position from it, so a decode step captured once in a HIP
  graph replays correctly at every position.  ``length`` is the host mirror.

``capacity`` is rounded up to a multiple of 32 (the attention kernel walks keys
in blocks of 32).  The buffers start zeroed, and only finite values are ever
appended, so the padding past ``length`` contributes exact zeros.
"""
from typing import List, Optional, Tuple

import torch

from . import _lib


def round_capacity(n: int) -> int:
    return max(32, (int(n) + 31) // 32 * 32)


class LayerKV:
    """View of one layer of a :class:`KVCache` (what ``past_key_value`` carries)."""

    def __init__(self, cache: "KVCache", layer: int):
        self.cache = cache
        self.layer = layer
        self.k = cache.k[layer]
        self.vt = cache.vt[layer]

    @property
    def length(self) -> int:
        return self.cache.length

    @property
    def counters(self) -> torch.Tensor:
        return self.cache.counters

    def as_tuple(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """``(k, v)`` in the reference layout ``[batch, kv_heads, length, head_dim]``."""
        n = self.cache.length
        return self.k[:, :, :n].contiguous(), self.vt[:, :, :, :n].transpose(2, 3).contiguous()


class KVCache:
    def __init__(self, num_layers: int, batch: int, num_kv_heads: int, head_dim: int, capacity: int,
                 device: Optional[torch.device] = None):
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.num_layers = num_layers
        self.batch = batch
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.capacity = round_capacity(capacity)
        self.device = device
        T = self.capacity
        self.k = torch.zeros((num_layers, batch, num_kv_heads, T, head_dim), dtype=torch.bfloat16, device=device)
        self.vt = torch.zeros((num_layers, batch, num_kv_heads, head_dim, T), dtype=torch.bfloat16, device=device)
        self.counters = torch.zeros(2, dtype=torch.int32, device=device)
        self.length = 0
        self.layers = [LayerKV(self, i) for i in range(num_layers)]

    def __getitem__(self, i: int) -> LayerKV:
        return self.layers[i]

    def __len__(self) -> int:
        return self.num_layers

    @property
    def nbytes(self) -> int:
        return 2 * self.k.numel() * self.k.element_size()

    def check_room(self, new_positions: int):
        if self.length + new_positions > self.capacity:
            raise RuntimeError(f"KV cache full: {self.length} + {new_positions} positions exceed capacity "
                               f"{self.capacity}")

    def advance(self, new_positions: int, steps: int = 0):
        """Account for ``new_positions`` appended by every layer (device counter and host mirror)."""
        self.check_room(new_positions)
        if steps and steps == new_positions:
            _lib.add_i32(self.counters, new_positions, n=2)
        else:
            _lib.add_i32(self.counters, new_positions, n=1)
            if steps:
                _lib.add_i32(self.counters[1:], steps, n=1)
        self.length += new_positions

    def reset(self):
        """Forget every cached position (the buffers are kept)."""
        self.counters.zero_()
        self.length = 0

    def load_tuples(self, past: List[Tuple[torch.Tensor, torch.Tensor]]):
        """Fill from reference-layout ``(k, v)`` pairs ``[batch, kv_heads, T, head_dim]``."""
        if len(past) != self.num_layers:
            raise ValueError(f"expected {self.num_layers} layers of cache, got {len(past)}")
        T = past[0][0].shape[2]
        if T > self.capacity:
            raise ValueError(f"{T} cached positions exceed capacity {self.capacity}")
        for i, (k, v) in enumerate(past):
            if k.shape != (self.batch, self.num_kv_heads, T, self.head_dim) or v.shape != k.shape:
                raise ValueError(f"layer {i}: cache tensors must be [batch, kv_heads, T, head_dim]")
            self.k[i, :, :, :T].copy_(k)
            self.vt[i, :, :, :, :T].copy_(v.transpose(2, 3))
        self.counters.copy_(torch.tensor([T, 0], dtype=torch.int32))
        self.length = T

    def as_tuples(self) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        return [layer.as_tuple() for layer in self.layers]
