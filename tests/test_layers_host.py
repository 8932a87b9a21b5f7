"""Host-side behaviour of the layer classes that needs no GPU: shard arithmetic and errors.

Mirrors the reference's shard-dimension tests (tests/test_parallel_layers.py:14-28, 91-101,
195-205) and the constructor / forward-before-load errors of
parallel/quantized_linear.py:71-74, 164-165, 203-204, 308-311, 431-432 and
parallel/embedding.py:239-242.
"""
import asyncio

import pytest

from shardcompute_amd.parallel import (ColumnParallelLinear, ParallelEmbedding, QuantizedColumnParallelLinear,
                                       QuantizedParallelEmbedding, QuantizedRowParallelLinear, RowParallelLinear,
                                       VocabParallelEmbedding)


def test_column_shard_dimensions():
    l0 = QuantizedColumnParallelLinear(256, 512, 2, 0)
    l1 = QuantizedColumnParallelLinear(256, 512, 2, 1)
    assert (l0.local_out_features, l0.col_start, l0.col_end) == (256, 0, 256)
    assert (l1.local_out_features, l1.col_start, l1.col_end) == (256, 256, 512)
    assert l0.num_parameters == 256 * 256 + 256
    assert l0.memory_bytes == 0


def test_row_shard_dimensions():
    l1 = QuantizedRowParallelLinear(512, 256, 2, 1)
    assert (l1.local_in_features, l1.row_start, l1.row_end) == (256, 256, 512)
    assert l1.num_parameters == 256 * 256  # bias only counted on rank 0
    assert QuantizedRowParallelLinear(512, 256, 2, 0).num_parameters == 256 * 256 + 256


def test_vocab_shard_dimensions():
    e = VocabParallelEmbedding(128256, 4096, 2, 0)
    assert (e.local_vocab_size, e.vocab_start, e.vocab_end) == (64128, 0, 64128)
    q = QuantizedParallelEmbedding(128256, 4096, 2, 1)
    assert (q.vocab_start, q.vocab_end) == (64128, 128256)
    p = ParallelEmbedding(1000, 256, 2, 1)
    assert (p.local_embedding_dim, p.col_start, p.col_end) == (128, 128, 256)


@pytest.mark.parametrize("ctor", [
    lambda: QuantizedColumnParallelLinear(256, 511, 2, 0),
    lambda: QuantizedRowParallelLinear(511, 256, 2, 0),
    lambda: ColumnParallelLinear(256, 511, 2, 0),
    lambda: RowParallelLinear(511, 256, 2, 0),
    lambda: VocabParallelEmbedding(1001, 64, 2, 0),
    lambda: QuantizedParallelEmbedding(1001, 64, 2, 0),
    lambda: ParallelEmbedding(1000, 65, 2, 0),
])
def test_divisibility_errors(ctor):
    with pytest.raises(ValueError):
        ctor()


def test_forward_before_load_raises():
    col = QuantizedColumnParallelLinear(64, 64, 1, 0)
    row = QuantizedRowParallelLinear(64, 64, 1, 0)
    with pytest.raises(RuntimeError):
        col.forward_sync(None)
    with pytest.raises(RuntimeError):
        asyncio.run(col.forward(None))
    with pytest.raises(RuntimeError):
        row.forward_partial(None)
    with pytest.raises(RuntimeError):
        asyncio.run(row.forward(None))
    with pytest.raises(RuntimeError):
        VocabParallelEmbedding(64, 8, 1, 0).forward_sync(None)


def test_repr_mentions_shard():
    assert "rank=1/2" in repr(QuantizedColumnParallelLinear(64, 128, 2, 1, bits=8))
    assert "bits=8" in repr(QuantizedRowParallelLinear(128, 64, 2, 1, bits=8))
