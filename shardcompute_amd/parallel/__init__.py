"""Tensor-parallel layer classes (one rank's shard) over the HIP kernels.

Mirrors the public classes of the reference's ``src/shardcompute/parallel/``.
"""
from .column_linear import ColumnParallelLinear
from .embedding import ParallelEmbedding, QuantizedParallelEmbedding, VocabParallelEmbedding
from .quantized_linear import QuantizedColumnParallelLinear, QuantizedRowParallelLinear
from .row_linear import FusedColumnRowLinear, RowParallelLinear

__all__ = [
    "ColumnParallelLinear", "RowParallelLinear", "FusedColumnRowLinear", "QuantizedColumnParallelLinear",
    "QuantizedRowParallelLinear",
    "ParallelEmbedding", "QuantizedParallelEmbedding", "VocabParallelEmbedding",
]
