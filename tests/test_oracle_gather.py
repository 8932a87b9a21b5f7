"""Pins oracle/gather.py (vocab-sharded masked gathers) and its C restatement."""
import numpy as np
import pytest

from oracle import cref
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.gather import qembed_gather_bf16, vocab_gather_bf16
from oracle.mlx_affine import dequantize_bf16, quantize_bf16


def _loop_gather(ids, table, start):
    """Per-token loop straight from embedding.py:325-356."""
    V, D = table.shape
    out = np.zeros((ids.size, D), np.uint16)
    for t, i in enumerate(np.asarray(ids).reshape(-1).tolist()):
        if start <= i < start + V:
            out[t] = table[i - start]
    return out.reshape(np.asarray(ids).shape + (D,))


def _special_table(rng, V, D):
    t = f32_to_bf16(rng.standard_normal((V, D)).astype(np.float32) * 0.02)
    t[1, :4] = [0x8000, 0x7FC1, 0x7F80, 0xFF80]  # -0.0, NaN with payload, +Inf, -Inf
    t[2, :] = 0x8000
    return t


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_gather_edges_and_dtypes(dtype):
    rng = np.random.default_rng(0)
    V, D, start = 50, 24, 100
    table = _special_table(rng, V, D)
    ids = np.array([[start - 1, start, start + 1, start + 2, start + V - 1, start + V, -1, -5000,
                     0, 10 ** 6]], dtype=dtype)
    got = vocab_gather_bf16(ids, table, start)
    assert np.array_equal(got, _loop_gather(ids, table, start))
    assert np.array_equal(got[0, 1], table[0]) and np.array_equal(got[0, 4], table[V - 1])
    assert np.array_equal(got[0, 2], table[1])  # -0.0 / NaN / Inf bits copied verbatim
    assert np.all(got[0, [0, 5, 6, 7, 8, 9]] == 0)  # out of shard -> +0.0


def test_gather_shards_sum_to_full_lookup():
    """The all-reduce (sum) of every rank's masked gather equals a plain take.

    Restates the reference's shard-vs-full lookup test
    (tests/test_parallel_layers.py:207-238) for the vocab-sharded layout.
    """
    rng = np.random.default_rng(1)
    V, D, ws = 96, 16, 3
    full = f32_to_bf16(rng.standard_normal((V, D)).astype(np.float32))
    ids = rng.integers(0, V, size=(4, 9))
    acc = np.zeros((4, 9, D), np.float32)
    for r in range(ws):
        lo = r * V // ws
        acc += bf16_to_f32(vocab_gather_bf16(ids, full[lo:lo + V // ws], lo))
    assert np.array_equal(acc, bf16_to_f32(np.take(full, ids, axis=0)))


@pytest.mark.parametrize("bits", [4, 8])
def test_qembed_gather(bits):
    rng = np.random.default_rng(2)
    V, D, start = 40, 128, 40
    w = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    wq, s, b = quantize_bf16(w, 64, bits)
    ids = np.array([39, 40, 41, 79, 80, 55, -1], np.int64)
    got = qembed_gather_bf16(ids, wq, s, b, start, 64, bits)
    deq = dequantize_bf16(wq, s, b, 64, bits)
    ref = _loop_gather(ids, deq, start)
    assert np.array_equal(got, ref)


@pytest.fixture(scope="module")
def clib():
    if not cref.available():
        cref.build()
    return cref.load()


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_c_gather_matches_numpy(clib, dtype):
    rng = np.random.default_rng(3)
    V, D, start = 300, 72, 300
    table = _special_table(rng, V, D)
    ids = rng.integers(-10, 700, size=(6, 33)).astype(dtype)
    assert np.array_equal(cref.vocab_gather_bf16(ids, table, start, threads=4),
                          vocab_gather_bf16(ids, table, start))
