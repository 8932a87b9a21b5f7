"""The public layer classes on the GPU against the oracle, through their own methods.

Each test drives a class the way the reference's callers do (constructor,
``load_*``, ``forward`` / ``forward_sync`` / ``forward_partial`` / ``add_bias``)
and compares with the oracle on the same packed weights:

* ``QuantizedColumnParallelLinear`` (``quantized_linear.py:17-251``): forward and
  forward_sync with a linear bias, ``gather_output`` through a communicator, the
  reference's errors, and ``load_shard_and_quantize``'s ``[in, local_out]``
  behaviour (``:96-125``: square shards give ``x @ W^T``, others fail);
* ``QuantizedRowParallelLinear`` (``:254-518``): ``forward_partial`` +
  ``add_bias`` against ``forward``, and the full-width scale/bias slicing of
  ``load_quantized_shard`` (``:385-414``) at world_size 8 for ranks 0 and 5:
  the rank's partial output is the oracle's product over its K slice (the
  rank-0 partial of a 70B-shape shard is exactly this path);
* dense ``ColumnParallelLinear`` / ``RowParallelLinear`` (``column_linear.py``,
  ``row_linear.py``, weights ``[in, out]``, ``x @ W``) and ``FusedColumnRowLinear``;
* ``ParallelEmbedding`` (``embedding.py:112-174``): dim-sharded lookup with
  ``padding_idx`` rows zeroed, bit for bit; ``VocabParallelEmbedding.load_shard``.

Bars: bit-exact for gathers and for identities between the classes' own
paths; LINEAR_TOL max-abs-rel against the oracle for products.
"""
import asyncio
import logging

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.gather import vocab_gather_bf16
from oracle.mlx_affine import quantize_bf16, quantized_matmul_bf16, quantized_matmul_f64
from shardcompute_amd.communicator import IdentityCommunicator
from shardcompute_amd.parallel import (ColumnParallelLinear, FusedColumnRowLinear, ParallelEmbedding,
                                       QuantizedColumnParallelLinear, QuantizedRowParallelLinear, RowParallelLinear,
                                       VocabParallelEmbedding)
from tests.gpu_util import LINEAR_TOL, dev, dev_bf16, host_u16, max_abs_rel

pytestmark = pytest.mark.gpu


def run(coro):
    return asyncio.run(coro)


def bf16_rand(rng, shape, scale=1.0):
    return f32_to_bf16((scale * rng.standard_normal(shape)).astype(np.float32))


def qweights(rng, n, k, bits, std=0.02):
    return quantize_bf16((std * rng.standard_normal((n, k))).astype(np.float32), 64, bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 5, 40])
def test_qcolumn_forward_bias_and_gather(device, bits, M):
    rng = np.random.default_rng(100 + bits + M)
    K, N, ws, rank = 512, 768, 2, 1
    wq, s, b = qweights(rng, N // ws, K, bits)
    bias = bf16_rand(rng, N // ws, 0.5)
    x = bf16_rand(rng, (2, M, K))
    comm = IdentityCommunicator(rank, ws)
    lin = QuantizedColumnParallelLinear(K, N, ws, rank, bias=True, gather_output=True, communicator=comm, bits=bits)
    assert (lin.local_out_features, lin.col_start, lin.col_end) == (N // 2, N // 2, N)
    lin.load_quantized_shard(wq, s, b, bias)
    y = run(lin.forward(dev_bf16(x)))
    assert comm.calls["all_gather"] == 1 and y.shape == (2, M, N // ws)
    ref = quantized_matmul_bf16(x.reshape(-1, K), wq, s, b, bias=bias, bits=bits)
    err = max_abs_rel(host_u16(y).reshape(-1, N // ws), ref)
    assert err <= LINEAR_TOL, err
    # forward_sync: the same product, no collective
    ys = lin.forward_sync(dev_bf16(x))
    assert torch.equal(ys, y) and comm.calls["all_gather"] == 1
    # without a bias: the bias-free product
    lin2 = QuantizedColumnParallelLinear(K, N, ws, rank, bias=False, bits=bits)
    lin2.load_quantized_shard(wq, s, b, bias)              # ignored: bias=False
    assert lin2.bias is None
    y2 = lin2.forward_sync(dev_bf16(x))
    assert max_abs_rel(host_u16(y2).reshape(-1, N // ws), quantized_matmul_bf16(x.reshape(-1, K), wq, s, b,
                                                                                  bits=bits)) <= LINEAR_TOL
    assert lin.memory_bytes == wq.nbytes + s.nbytes + b.nbytes + bias.nbytes
    assert lin.num_parameters == K * (N // ws) + N // ws


def test_qcolumn_errors(device):
    with pytest.raises(ValueError):
        QuantizedColumnParallelLinear(512, 100, 3, 0)
    lin = QuantizedColumnParallelLinear(512, 256, 1, 0, gather_output=True, communicator=None)
    x = torch.zeros((1, 512), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="not loaded"):
        run(lin.forward(x))
    with pytest.raises(RuntimeError, match="not loaded"):
        lin.forward_sync(x)
    rng = np.random.default_rng(7)
    lin.load_quantized_shard(*qweights(rng, 256, 512, 4))
    with pytest.raises(RuntimeError, match="Communicator required"):
        run(lin.forward(x))
    with pytest.raises(ValueError):
        lin.load_shard_and_quantize(np.zeros((256, 512), np.float32))   # expects [in, local_out]


def test_qcolumn_load_shard_and_quantize(device):
    # the reference quantizes the [in, local_out] shard along local_out and then
    # multiplies with transpose=True: a square shard W gives x @ Wq^T, where Wq is
    # W quantized along its rows; a non-square shard cannot be applied to x
    rng = np.random.default_rng(8)
    n = 256
    w = (0.02 * rng.standard_normal((n, n))).astype(np.float32)
    lin = QuantizedColumnParallelLinear(n, n, 1, 0, bias=False)
    lin.load_shard_and_quantize(w)
    wq, s, b = quantize_bf16(w, 64, 4)
    assert np.array_equal(host_u16(lin.scales), s) and np.array_equal(host_u16(lin.biases_quant), b)
    x = bf16_rand(rng, (3, n))
    y = lin.forward_sync(dev_bf16(x))
    assert max_abs_rel(host_u16(y), quantized_matmul_bf16(x, wq, s, b)) <= LINEAR_TOL
    # the product is x @ W^T (rows of the given [in, out] matrix act as outputs):
    # within 4-bit quantization noise of it, and nowhere near x @ W
    xf = bf16_to_f32(x).astype(np.float64)
    assert max_abs_rel(host_u16(y), xf @ w.astype(np.float64).T) <= 0.2
    assert max_abs_rel(host_u16(y), xf @ w.astype(np.float64)) >= 0.8
    rect = QuantizedColumnParallelLinear(128, 256, 1, 0, bias=False)
    rect.load_shard_and_quantize((0.02 * rng.standard_normal((128, 256))).astype(np.float32))
    with pytest.raises(ValueError):
        rect.forward_sync(dev_bf16(bf16_rand(rng, (1, 128))))


@pytest.mark.parametrize("bits", [4, 8])
def test_qrow_partial_bias_and_forward(device, bits):
    rng = np.random.default_rng(200 + bits)
    K, N = 1024, 512
    wq, s, b = qweights(rng, N, K, bits)
    bias = bf16_rand(rng, N, 0.5)
    x = bf16_rand(rng, (4, K))
    lin = QuantizedRowParallelLinear(K, N, 1, 0, bias=True, bits=bits)
    lin.load_quantized_shard(wq, s, b, bias)
    part = lin.forward_partial(dev_bf16(x))
    assert max_abs_rel(host_u16(part), quantized_matmul_bf16(x, wq, s, b, bits=bits)) <= LINEAR_TOL
    full = lin.add_bias(part)
    assert max_abs_rel(host_u16(full), quantized_matmul_bf16(x, wq, s, b, bias=bias, bits=bits)) <= LINEAR_TOL
    # forward (identity all-reduce, bias fused into the product's epilogue) equals
    # partial -> all-reduce -> add_bias bit for bit
    fwd = run(lin.forward(dev_bf16(x)))
    assert torch.equal(fwd, full)
    comm = IdentityCommunicator(0, 1)
    lin.communicator = comm
    assert torch.equal(run(lin.forward(dev_bf16(x))), full)
    # bias only on rank 0
    r1 = QuantizedRowParallelLinear(2 * K, N, 2, 1, bias=True, bits=bits)
    r1.load_quantized_shard(wq, s, b, bias)
    assert r1.bias is None and torch.equal(r1.add_bias(part), part)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rank", [0, 5])
def test_qrow_full_width_scale_slicing(device, bits, rank, caplog):
    # world_size 8: the weight shard holds this rank's K slice, scales/biases are
    # supplied for every rank's groups (as a full-width checkpoint stores them)
    rng = np.random.default_rng(300 + 10 * bits + rank)
    ws, N, K = 8, 256, 8 * 512
    wq_f, s_f, b_f = qweights(rng, N, K, bits)
    kl = K // ws
    wpk = kl * bits // 32
    gl = kl // 64
    wq_r = np.ascontiguousarray(wq_f[:, rank * wpk:(rank + 1) * wpk])
    lin = QuantizedRowParallelLinear(K, N, ws, rank, bias=True, bits=bits)
    assert (lin.local_in_features, lin.row_start, lin.row_end) == (kl, rank * kl, (rank + 1) * kl)
    lin.load_quantized_shard(wq_r, s_f, b_f, bf16_rand(rng, N))
    assert lin.scales.shape == (N, gl) and lin.biases_quant.shape == (N, gl)
    assert np.array_equal(host_u16(lin.scales), s_f[:, rank * gl:(rank + 1) * gl])
    assert np.array_equal(host_u16(lin.biases_quant), b_f[:, rank * gl:(rank + 1) * gl])
    assert (lin.bias is not None) == (rank == 0)
    x_full = bf16_rand(rng, (3, K))
    x_r = np.ascontiguousarray(x_full[:, rank * kl:(rank + 1) * kl])
    part = lin.forward_partial(dev_bf16(x_r))
    ref = quantized_matmul_f64(x_r, wq_r, s_f[:, rank * gl:(rank + 1) * gl], b_f[:, rank * gl:(rank + 1) * gl],
                               bits=bits)
    assert max_abs_rel(host_u16(part), ref) <= LINEAR_TOL
    # the eight ranks' partials sum to the full product (the all-reduce's result)
    if rank == 0:
        tot = np.zeros((3, N))
        for r in range(ws):
            lr = QuantizedRowParallelLinear(K, N, ws, r, bias=False, bits=bits)
            lr.load_quantized_shard(np.ascontiguousarray(wq_f[:, r * wpk:(r + 1) * wpk]), s_f, b_f)
            tot += bf16_to_f32(host_u16(lr.forward_partial(
                dev_bf16(np.ascontiguousarray(x_full[:, r * kl:(r + 1) * kl]))))).astype(np.float64)
        full = quantized_matmul_f64(x_full, wq_f, s_f, b_f, bits=bits)
        assert np.abs(tot - full).max() / np.abs(full).max() <= 2 * LINEAR_TOL
    # scales already local: unchanged; a width that matches neither: unchanged, with the warning
    lin2 = QuantizedRowParallelLinear(K, N, ws, rank, bias=False, bits=bits)
    s_loc = np.ascontiguousarray(s_f[:, :gl])
    lin2.load_quantized_shard(wq_r, s_loc, np.ascontiguousarray(b_f[:, :gl]))
    assert np.array_equal(host_u16(lin2.scales), s_loc)
    lin3 = QuantizedRowParallelLinear(K, N, ws, rank, bias=False, bits=bits)
    with caplog.at_level(logging.WARNING):
        lin3.load_quantized_shard(wq_r, np.ascontiguousarray(s_f[:, :3 * gl]), np.ascontiguousarray(b_f[:, :3 * gl]))
    assert lin3.scales.shape == (N, 3 * gl)
    assert any("does not match expected groups" in r.getMessage() for r in caplog.records)


def test_qrow_load_shard_and_quantize(device):
    rng = np.random.default_rng(9)
    n = 256
    w = (0.02 * rng.standard_normal((n, n))).astype(np.float32)
    lin = QuantizedRowParallelLinear(n, n, 1, 0, bias=True)
    bias = bf16_rand(rng, n)
    lin.load_shard_and_quantize(w, bias)
    wq, s, b = quantize_bf16(w, 64, 4)
    x = bf16_rand(rng, (2, n))
    y = run(lin.forward(dev_bf16(x)))
    assert max_abs_rel(host_u16(y), quantized_matmul_bf16(x, wq, s, b, bias=bias)) <= LINEAR_TOL
    with pytest.raises(ValueError):
        lin.load_shard_and_quantize(np.zeros((n, 2 * n), np.float32))


def _dense64(x_u16, w_u16):
    return bf16_to_f32(x_u16).astype(np.float64) @ bf16_to_f32(w_u16).astype(np.float64)


def test_dense_column_row_forward(device):
    # weights in the reference's [in, out] layout: y = x @ W (column_linear.py:155, row_linear.py:163)
    rng = np.random.default_rng(10)
    K, N, ws = 256, 384, 2
    W = bf16_rand(rng, (K, N), 0.05)
    bias = bf16_rand(rng, N, 0.5)
    x = bf16_rand(rng, (2, 3, K))
    for rank in range(ws):
        col = ColumnParallelLinear(K, N, ws, rank, bias=True, gather_output=False)
        col.load_shard(dev_bf16(W), dev_bf16(bias))
        c0, c1 = rank * N // ws, (rank + 1) * N // ws
        y = run(col.forward(dev_bf16(x)))
        ref = _dense64(x.reshape(-1, K), W[:, c0:c1]) + bf16_to_f32(bias[c0:c1])
        assert max_abs_rel(host_u16(y).reshape(-1, c1 - c0), ref) <= LINEAR_TOL
        assert torch.equal(col.forward_sync(dev_bf16(x)), y)
    # load_shard_direct with a pre-sharded [in, local_out] matrix and its bias
    col = ColumnParallelLinear(K, N, 1, 0, bias=True, gather_output=True, communicator=IdentityCommunicator())
    col.load_shard_direct(dev_bf16(W), dev_bf16(bias))
    y = run(col.forward(dev_bf16(x)))
    assert max_abs_rel(host_u16(y).reshape(-1, N), _dense64(x.reshape(-1, K), W) + bf16_to_f32(bias)) <= LINEAR_TOL
    # row parallel: each rank's [K/ws, N] rows on its input slice; partials sum to the
    # full product, bias once (rank 0)
    tot = np.zeros((6, N))
    for rank in range(ws):
        row = RowParallelLinear(K, N, ws, rank, bias=True)
        row.load_shard(dev_bf16(W), dev_bf16(bias))
        r0, r1 = rank * K // ws, (rank + 1) * K // ws
        xs = np.ascontiguousarray(x[..., r0:r1])
        p = row.forward_partial(dev_bf16(xs))
        assert max_abs_rel(host_u16(p).reshape(-1, N), _dense64(xs.reshape(-1, r1 - r0), W[r0:r1])) <= LINEAR_TOL
        tot += bf16_to_f32(host_u16(p).reshape(-1, N))
        out = run(row.forward(dev_bf16(xs)))
        assert (row.bias is not None) == (rank == 0)
        assert torch.equal(out, row.add_bias(p))
    ref = _dense64(x.reshape(-1, K), W) + bf16_to_f32(bias)
    assert np.abs(tot + bf16_to_f32(bias) - ref).max() / np.abs(ref).max() <= 2 * LINEAR_TOL
    with pytest.raises(ValueError):
        RowParallelLinear(K, N, ws, 0).load_shard_direct(dev_bf16(W))


@pytest.mark.parametrize("activation", ["silu", "gelu", "relu"])
def test_fused_column_row(device, activation):
    rng = np.random.default_rng(11)
    K, Hd, N = 128, 256, 128
    up, down = bf16_rand(rng, (K, Hd), 0.1), bf16_rand(rng, (Hd, N), 0.1)
    ub, db = bf16_rand(rng, Hd, 0.1), bf16_rand(rng, N, 0.1)
    f = FusedColumnRowLinear(K, Hd, N, 1, 0, activation=activation, bias=True, communicator=IdentityCommunicator())
    f.load_shards(dev_bf16(up), dev_bf16(ub), dev_bf16(down), dev_bf16(db))
    x = bf16_rand(rng, (4, K))
    y = run(f.forward(dev_bf16(x)))
    h = _dense64(x, up) + bf16_to_f32(ub)
    act = {"silu": lambda v: v / (1 + np.exp(-v)), "gelu": lambda v: v / (1 + np.exp(-1.702 * v)),
           "relu": lambda v: np.maximum(v, 0)}[activation](h)
    ref = act @ bf16_to_f32(down).astype(np.float64) + bf16_to_f32(db)
    assert max_abs_rel(host_u16(y), ref) <= 2 * LINEAR_TOL


@pytest.mark.parametrize("ids_dtype", [np.int32, np.int64])
def test_parallel_embedding_padding_idx(device, ids_dtype):
    rng = np.random.default_rng(12)
    V, D, ws, pad = 500, 256, 2, 7
    table = bf16_rand(rng, (V, D))
    table[pad] = f32_to_bf16(np.full(D, 3.0, np.float32))    # a nonzero row that padding must hide
    ids = rng.integers(0, V, (3, 40)).astype(ids_dtype)
    ids[0, :5] = pad
    ids[2, -1] = V - 1
    for rank in range(ws):
        comm = IdentityCommunicator(rank, ws)
        e = ParallelEmbedding(V, D, ws, rank, gather_output=True, communicator=comm, padding_idx=pad)
        e.load_shard(dev_bf16(table))
        c0, c1 = rank * D // ws, (rank + 1) * D // ws
        got = host_u16(run(e.forward(dev(ids))))
        ref = vocab_gather_bf16(ids, np.ascontiguousarray(table[:, c0:c1]), 0)
        ref[ids == pad] = 0
        assert got.shape == (3, 40, D // ws)
        assert np.array_equal(got, ref)
        assert comm.calls["all_gather"] == 1
        assert np.array_equal(host_u16(e.forward_sync(dev(ids))), ref)
    # without padding_idx the row is returned as stored
    e = ParallelEmbedding(V, D, 1, 0, gather_output=False)
    e.load_shard_direct(dev_bf16(table))
    assert np.array_equal(host_u16(run(e.forward(dev(ids)))), vocab_gather_bf16(ids, table, 0))
    with pytest.raises(RuntimeError, match="Communicator required"):
        g = ParallelEmbedding(V, D, 1, 0, gather_output=True, communicator=None)
        g.load_shard_direct(dev_bf16(table))
        run(g.forward(dev(ids)))


def test_vocab_embedding_load_shard(device):
    rng = np.random.default_rng(13)
    V, D, ws = 640, 128, 4
    table = bf16_rand(rng, (V, D))
    ids = rng.integers(-3, V + 3, (2, 50)).astype(np.int64)
    parts = []
    for rank in range(ws):
        e = VocabParallelEmbedding(V, D, ws, rank, communicator=IdentityCommunicator(rank, ws))
        e.load_shard(dev_bf16(table))
        got = host_u16(run(e.forward(dev(ids))))
        assert np.array_equal(got, vocab_gather_bf16(ids, table[e.vocab_start:e.vocab_end], e.vocab_start))
        parts.append(bf16_to_f32(got))
    # the ranks' masked rows sum (the all-reduce) to the full lookup, ids out of range zero
    full = vocab_gather_bf16(ids, table, 0)
    assert np.array_equal(f32_to_bf16(np.sum(parts, axis=0).astype(np.float32)), full)
