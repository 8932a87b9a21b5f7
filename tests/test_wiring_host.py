"""Host-side logic of the decoder wiring (no GPU needed)."""
import asyncio

import numpy as np
import pytest
import torch

from oracle.decoder import rope_cos_sin
from shardcompute_amd.communicator import IdentityCommunicator
from shardcompute_amd.executor import ExecutionMetrics, LayerTiming
from shardcompute_amd.kv_cache import KVCache, round_capacity
from shardcompute_amd.parallel.attention import ParallelAttention, RoPE, rope_tables_np
from shardcompute_amd.parallel.mlp import ParallelMLP
from shardcompute_amd.parallel.transformer import ParallelTransformer, run_sync


def test_rope_tables_match_oracle_and_closed_form():
    for D, base in ((64, 10000.0), (128, 500000.0)):
        c, s = rope_tables_np(D, base, 1.0, 3000)
        oc, os_ = rope_cos_sin(np.arange(3000), D, base)
        assert np.array_equal(c, oc[:, :D // 2]) and np.array_equal(s, os_[:, :D // 2])
        # closed form in fp64: angle t * base^(-2i/D); fp32 angles lose ~t * 2^-24 rad
        t = np.arange(3000)[:, None].astype(np.float64)
        ang = t * base ** (-np.arange(0, D, 2) / D)[None, :]
        tol = 3000 * 2.0 ** -22
        assert np.abs(c - np.cos(ang)).max() < tol and np.abs(s - np.sin(ang)).max() < tol


def test_rope_scaling_factor_divides_positions():
    c1, _ = rope_tables_np(64, 10000.0, 2.0, 300)
    c2, _ = rope_tables_np(64, 10000.0, 1.0, 200)
    assert np.array_equal(c1[100], c2[50]) and np.array_equal(c1[2 * 37], c2[37])
    r = RoPE(64, max_position_embeddings=128, base=10000.0)
    assert r.inv_freq.dtype == np.float32 and r.inv_freq.shape == (32,)


def test_run_sync():
    async def f(x):
        await IdentityCommunicator().all_reduce(None)
        return x + 1
    assert run_sync(f(2)) == 3

    async def g():
        await asyncio.sleep(0)
    with pytest.raises(RuntimeError, match="suspended"):
        run_sync(g())


def test_attention_constructor_validation():
    a = ParallelAttention(4096, 32, 1, 0, None, num_kv_heads=8, use_quantized=True)
    assert a.head_dim == 128 and a.local_num_kv_heads == 8 and a.qkv_width == (32 + 16) * 128
    assert a.scale == pytest.approx(1 / np.sqrt(128))
    s = ParallelAttention(8192, 64, 8, 0, None, num_kv_heads=8, use_quantized=True)
    assert s.local_num_heads == 8 and s.local_num_kv_heads == 1 and s.qkv_width == 10 * 128
    with pytest.raises(ValueError):
        ParallelAttention(4096, 30, 4, 0, None)
    with pytest.raises(ValueError):
        ParallelAttention(4096, 32, 4, 0, None, num_kv_heads=2)
    with pytest.raises(RuntimeError):
        a2 = ParallelAttention(256, 4, 1, 0, None)
        a2.load_quantized_shards(*([None] * 16))
    # the additive attention mask's broadcast view (what the masked kernel reads)
    from shardcompute_amd._lib import broadcast_mask
    m = broadcast_mask(torch.zeros((4, 9)), 2, 8, 4, 9)
    assert m.shape == (2, 8, 4, 9) and m.stride() == (0, 0, 9, 1) and m.dtype == torch.float32
    m = broadcast_mask(torch.zeros((2, 1, 1, 9), dtype=torch.bfloat16), 2, 8, 4, 9)
    assert m.stride() == (9, 0, 0, 1) and m.dtype == torch.float32
    with pytest.raises(ValueError, match="does not broadcast"):
        broadcast_mask(torch.zeros((3, 9)), 2, 8, 4, 9)
    with pytest.raises(ValueError, match="n_keys"):
        broadcast_mask(torch.zeros((4, 9)), 2, 8, 4, None)


def test_mlp_constructor_validation():
    m = ParallelMLP(4096, 14336, 1, 0, None, use_quantized=True)
    assert m.local_intermediate == 14336 and m.gate_up is not None
    with pytest.raises(ValueError):
        ParallelMLP(4096, 14335, 2, 0, None)
    with pytest.raises(ValueError):
        ParallelMLP(4096, 14336, 1, 0, None, activation="tanhh")
    # every activation the reference accepts constructs, gated or not; only the gated
    # SiLU runs fused into the gate|up product
    for act in ("silu", "swish", "gelu", "gelu_new", "relu", "gelu_exact"):
        for gated in (True, False):
            g = ParallelMLP(64, 128, 1, 0, None, activation=act, use_gated=gated, use_quantized=True)
            assert g.fused_swiglu == (gated and act in ("silu", "swish"))
            assert (g.gate_up is None) == (not gated)
    with pytest.raises(RuntimeError, match="Weight not loaded"):
        ParallelMLP(64, 128, 1, 0, None, activation="gelu", use_quantized=True).intermediate(torch.zeros(1, 64))


def test_transformer_construction_defaults():
    t = ParallelTransformer(1000, 256, 2, 4, 512, 1, 0, use_quantized=True)
    assert type(t.embed_tokens).__name__ == "QuantizedParallelEmbedding"
    assert type(t.lm_head).__name__ == "ColumnParallelLinear"
    assert isinstance(t.communicator, IdentityCommunicator)
    t2 = ParallelTransformer(1000, 256, 2, 4, 512, 1, 0, use_quantized=True, embedding="vocab",
                             quantized_lm_head=True)
    assert type(t2.embed_tokens).__name__ == "VocabParallelEmbedding"
    assert type(t2.lm_head).__name__ == "QuantizedColumnParallelLinear"
    t3 = ParallelTransformer(1000, 256, 2, 4, 512, 1, 0)
    assert type(t3.embed_tokens).__name__ == "ParallelEmbedding"
    with pytest.raises(ValueError):
        ParallelTransformer(1000, 256, 2, 4, 512, 1, 0, embedding="sparse")
    with pytest.raises(IndexError):
        t.get_layer(2)
    with pytest.raises(RuntimeError):
        t3.load_quantized_embedding_weights(None, None, None)


def test_kv_cache_layout_roundtrip():
    assert round_capacity(1) == 32 and round_capacity(33) == 64 and round_capacity(64) == 64
    c = KVCache(2, 3, 2, 16, 40, device=torch.device("cpu"))
    assert c.capacity == 64 and c.k.shape == (2, 3, 2, 64, 16) and c.vt.shape == (2, 3, 2, 16, 64)
    g = torch.Generator().manual_seed(0)
    past = [(torch.randn(3, 2, 10, 16, generator=g).bfloat16(), torch.randn(3, 2, 10, 16, generator=g).bfloat16())
            for _ in range(2)]
    c.load_tuples(past)
    assert c.length == 10 and c.counters.tolist() == [10, 0]
    for (k0, v0), (k1, v1) in zip(past, c.as_tuples()):
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
    assert torch.equal(c.vt[0, :, :, :, :10], past[0][1].transpose(2, 3))
    c.check_room(54)
    with pytest.raises(RuntimeError, match="full"):
        c.check_room(55)
    with pytest.raises(ValueError):
        c.load_tuples(past[:1])


def test_execution_metrics():
    # LayerTiming(layer_idx, layer_type, compute_ms, comm_ms) as worker/executor.py:19-29
    m = ExecutionMetrics(total_time_ms=10.0, layer_timings=[LayerTiming(-1, "embedding", 0.5),
                                                            LayerTiming(0, "transformer", 3.0, 1.0),
                                                            LayerTiming(1, "transformer", 5.0, 1.0)],
                         input_tokens=4, output_shape=[1, 4])
    assert m.compute_time_ms == 8.5 and m.comm_time_ms == 2.0 and m.compute_fraction == pytest.approx(8.5 / 10.5)
    d = m.to_dict()
    assert d["num_layers"] == 2
    assert d["layer_timings"][2] == {"layer": 1, "type": "transformer", "compute_ms": 5.0, "comm_ms": 1.0}
