"""Dense row-parallel linear (``src/shardcompute/parallel/row_linear.py:12-217``)
and the column -> activation -> row composition ``FusedColumnRowLinear``
(``:220-311``).

Not a hot-path kernel: ``[local_in, out]`` weights, torch GEMM, all-reduce
through the communicator when one is given, bias on rank 0 only.
"""
import logging
from typing import Optional

import torch

from ._tensors import default_device, to_device

logger = logging.getLogger(__name__)


class RowParallelLinear:
    def __init__(self, in_features: int, out_features: int, world_size: int, rank: int, bias: bool = True,
                 input_is_partitioned: bool = True, communicator=None, device=None):
        self.in_features = in_features
        self.out_features = out_features
        self.world_size = world_size
        self.rank = rank
        self.input_is_partitioned = input_is_partitioned
        self.communicator = communicator
        if in_features % world_size != 0:
            raise ValueError(f"in_features ({in_features}) must be divisible by world_size ({world_size})")
        self.local_in_features = in_features // world_size
        self.row_start = rank * self.local_in_features
        self.row_end = self.row_start + self.local_in_features
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
        self.weight = w[self.row_start:self.row_end, :].contiguous()
        if self.has_bias and full_bias is not None and self.rank == 0:
            self.bias = to_device(full_bias, self.device, torch.bfloat16)

    def load_shard_direct(self, weight_shard, bias_shard=None):
        if weight_shard is None:
            logger.warning("load_shard_direct called with None weight, skipping")
            return
        expected = (self.local_in_features, self.out_features)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}")
        self.weight = to_device(weight_shard, self.device, torch.bfloat16)
        if self.has_bias and bias_shard is not None and self.rank == 0:
            self.bias = to_device(bias_shard, self.device, torch.bfloat16)

    def forward_partial(self, x):
        if self.weight is None:
            raise RuntimeError("Weight not loaded")
        return x @ self.weight

    def add_bias(self, x):
        if self.has_bias and self.bias is not None:
            return x + self.bias
        return x

    async def forward(self, x):
        out = self.forward_partial(x)
        if self.communicator is not None:
            out = await self.communicator.all_reduce(out, op="sum")
        return self.add_bias(out)

    @property
    def num_parameters(self) -> int:
        return self.local_in_features * self.out_features + (
            self.out_features if self.has_bias and self.rank == 0 else 0)

    def __repr__(self):
        return (f"RowParallelLinear(in_features={self.in_features}, out_features={self.out_features}, "
                f"local_in_features={self.local_in_features}, rank={self.rank}/{self.world_size})")


def _activation(name):
    """The activations of ``row_linear.py:268-276``, on bf16 tensors computed in fp32."""
    if name == "gelu":
        return lambda x: (x.float() * torch.sigmoid(1.702 * x.float())).to(x.dtype)   # sigmoid approximation
    if name in ("silu", "swish"):
        return lambda x: (x.float() * torch.sigmoid(x.float())).to(x.dtype)
    if name == "relu":
        return lambda x: torch.clamp_min(x, 0)
    return lambda x: x


class FusedColumnRowLinear:
    """Column-parallel up projection -> activation -> row-parallel down projection
    with one all-reduce at the end (``row_linear.py:220-311``).

    The reference module refers to ``ColumnParallelLinear`` without importing it,
    so its constructor raises ``NameError`` as shipped; this class builds what the
    constructor describes: ``up_proj`` a ``ColumnParallelLinear`` (no gather, no
    communicator), ``down_proj`` a ``RowParallelLinear`` carrying the
    communicator.  Dense ``[in, out]`` weights and torch GEMMs, as the two
    classes it composes."""

    def __init__(self, in_features: int, hidden_features: int, out_features: int, world_size: int, rank: int,
                 activation: str = "gelu", bias: bool = True, communicator=None, device=None):
        from .column_linear import ColumnParallelLinear
        self.in_features = in_features
        self.hidden_features = hidden_features
        self.out_features = out_features
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        self.up_proj = ColumnParallelLinear(in_features, hidden_features, world_size, rank, bias=bias,
                                            gather_output=False, communicator=None, device=device)
        self.down_proj = RowParallelLinear(hidden_features, out_features, world_size, rank, bias=bias,
                                           input_is_partitioned=True, communicator=communicator, device=device)
        self.activation_name = activation
        self.activation = _activation(activation)

    def load_shards(self, up_weight, up_bias, down_weight, down_bias):
        self.up_proj.load_shard_direct(up_weight, up_bias)
        self.down_proj.load_shard_direct(down_weight, down_bias)

    async def forward(self, x):
        hidden = self.activation(self.up_proj.forward_sync(x))
        return await self.down_proj.forward(hidden)
