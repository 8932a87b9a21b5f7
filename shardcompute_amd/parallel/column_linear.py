"""Dense column-parallel linear (``src/shardcompute/parallel/column_linear.py:12-208``).

Not a hot-path kernel: weights keep the reference's ``[in, local_out]`` layout
and the product is torch's GEMM on the GPU.  Kept so a model that mixes dense
and quantized projections (e.g. a dense lm_head) loads unchanged.
"""
import logging
from typing import Optional

import torch

from ._tensors import default_device, to_device

logger = logging.getLogger(__name__)


class ColumnParallelLinear:
    def __init__(self, in_features: int, out_features: int, world_size: int, rank: int, bias: bool = True,
                 gather_output: bool = False, communicator=None, device=None):
        self.in_features = in_features
        self.out_features = out_features
        self.world_size = world_size
        self.rank = rank
        self.gather_output = gather_output
        self.communicator = communicator
        if out_features % world_size != 0:
            raise ValueError(f"out_features ({out_features}) must be divisible by world_size ({world_size})")
        self.local_out_features = out_features // world_size
        self.col_start = rank * self.local_out_features
        self.col_end = self.col_start + self.local_out_features
        self.weight: Optional[torch.Tensor] = None
        self.bias: Optional[torch.Tensor] = None
        self.has_bias = bias
        self._device = device

    @property
    def device(self):
        if self._device is None:
            self._device = default_device()
        return self._device

    def load_shard(self, full_weight, full_bias=None):
        w = to_device(full_weight, self.device, torch.bfloat16)
        self.weight = w[:, self.col_start:self.col_end].contiguous()
        if self.has_bias and full_bias is not None:
            self.bias = to_device(full_bias, self.device, torch.bfloat16)[self.col_start:self.col_end].contiguous()

    def load_shard_direct(self, weight_shard, bias_shard=None):
        if weight_shard is None:
            logger.warning("load_shard_direct called with None weight, skipping")
            return
        expected = (self.in_features, self.local_out_features)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}")
        self.weight = to_device(weight_shard, self.device, torch.bfloat16)
        if self.has_bias and bias_shard is not None:
            self.bias = to_device(bias_shard, self.device, torch.bfloat16)

    def _mm(self, x):
        out = x @ self.weight
        if self.has_bias and self.bias is not None:
            out = out + self.bias
        return out

    async def forward(self, x):
        if self.weight is None:
            raise RuntimeError("Weight not loaded. Call load_shard() or load_shard_direct() first.")
        out = self._mm(x)
        if self.gather_output:
            if self.communicator is None:
                raise RuntimeError("Communicator required for gather_output=True")
            out = await self.communicator.all_gather(out, dim=-1)
        return out

    def forward_sync(self, x):
        if self.weight is None:
            raise RuntimeError("Weight not loaded")
        return self._mm(x)

    @property
    def num_parameters(self) -> int:
        return self.in_features * self.local_out_features + (self.local_out_features if self.has_bias else 0)

    def __repr__(self):
        return (f"ColumnParallelLinear(in_features={self.in_features}, out_features={self.out_features}, "
                f"local_out_features={self.local_out_features}, rank={self.rank}/{self.world_size}, "
                f"bias={self.has_bias})")
