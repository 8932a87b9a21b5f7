"""Vocab-sharded masked row gathers, restated in numpy — TEST INFRASTRUCTURE ONLY.

Follows ``QuantizedParallelEmbedding.forward``
(``src/shardcompute/parallel/embedding.py:322-356``):

    local_ids = input_ids - vocab_start                       # :325
    in_range  = (input_ids >= vocab_start) & (input_ids < vocab_end)   # :328
    local_ids = clip(local_ids, 0, local_vocab_size - 1)     # :331
    rows      = take(table, local_ids, axis=0)                # :338-340
    (dequantize for the quantized table)                      # :343-349
    out       = where(in_range, rows, zeros_like(rows))       # :356

``VocabParallelEmbedding`` (``embedding.py:397-418``) is a stub in the
reference; the HIP library implements these mask semantics on a bf16 table,
which is ``vocab_gather_bf16`` here.  Zero rows are +0.0 (``mx.zeros_like``).

Parity: the semantics are plain index arithmetic; the tests pin them against
``np.take`` + an explicit per-token loop, at the shard edges
(``vocab_start - 1``, ``vocab_start``, ``vocab_end - 1``, ``vocab_end``),
negative ids, int32 and int64 ids, and rows holding -0.0 / NaN / Inf bit
patterns (copied verbatim).  The reference's own tests pin only the dense
``mx.take`` path (``tests/test_parallel_layers.py:207-238``: shard concat ==
full lookup), which ``test_oracle_gather.py`` restates.
"""
import numpy as np

from .mlx_affine import dequantize_bf16


def in_shard_mask(ids, vocab_start, vocab_end):
    ids = np.asarray(ids).astype(np.int64)
    return (ids >= vocab_start) & (ids < vocab_end)


def vocab_gather_bf16(ids, table, vocab_start):
    """ids int [..], table uint16 [V_local, D] -> uint16 [.., D] (bit-exact)."""
    table = np.asarray(table)
    ids64 = np.asarray(ids).astype(np.int64)
    v_local = table.shape[0]
    local = np.clip(ids64 - vocab_start, 0, v_local - 1)
    rows = np.take(table, local.reshape(-1), axis=0)
    keep = in_shard_mask(ids64, vocab_start, vocab_start + v_local).reshape(-1)
    rows = np.where(keep[:, None], rows, np.zeros_like(rows))
    return rows.reshape(ids64.shape + (table.shape[1],))


def qembed_gather_bf16(ids, wq, scales, biases, vocab_start, group_size=64, bits=4):
    """Masked gather of a quantized table, dequantized to bf16 (uint16).

    Each in-shard row is ``dequantize_bf16`` of the selected (wq, s, b) row;
    out-of-shard rows are +0.0.
    """
    ids64 = np.asarray(ids).astype(np.int64)
    wq = np.asarray(wq)
    v_local = wq.shape[0]
    local = np.clip(ids64 - vocab_start, 0, v_local - 1).reshape(-1)
    rows = dequantize_bf16(wq[local], np.asarray(scales)[local], np.asarray(biases)[local],
                           group_size, bits)
    keep = in_shard_mask(ids64, vocab_start, vocab_start + v_local).reshape(-1)
    rows = np.where(keep[:, None], rows, np.zeros_like(rows))
    return rows.reshape(ids64.shape + (rows.shape[1],))
