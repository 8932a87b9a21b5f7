"""ModelLoader key mapping on the CPU, against a recording stand-in model.

Shard files follow the reference layout (``rank_<r>/model.safetensors``,
Hugging Face names, ``src/shardcompute/model/loader.py:106-413``); the stand-in
records which loader method received which tensors, so the mapping (Llama and
Phi-2 names, quantized and dense paths, the shared-layernorm fallback) is checked
without a GPU.
"""
import asyncio
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from shardcompute_amd.loader import ModelLoader, detect_parallelism_mode


class Rec:
    """Records calls as (name, args, kwargs)."""

    def __init__(self, log, name):
        self._log, self._name = log, name

    def __getattr__(self, attr):
        if attr.startswith("_"):
            raise AttributeError(attr)

        def call(*a, **k):
            self._log.append((f"{self._name}.{attr}", a, k))
        return call


class FakeLayer:
    def __init__(self, log, i):
        self.input_layernorm = Rec(log, f"layers.{i}.input_layernorm")
        self.post_attention_layernorm = Rec(log, f"layers.{i}.post_attention_layernorm")
        self.attention = Rec(log, f"layers.{i}.attention")
        self.mlp = Rec(log, f"layers.{i}.mlp")


class FakeModel:
    def __init__(self, n_layers, lm_quantized=True):
        self.log = []
        self.layers = [FakeLayer(self.log, i) for i in range(n_layers)]
        self.embed_tokens = Rec(self.log, "embed_tokens")
        self.norm = Rec(self.log, "norm")
        self.lm_head = Rec(self.log, "lm_head")
        if not lm_quantized:
            self.lm_head = _DenseHead(self.log)

    def load_quantized_embedding_weights(self, *a):
        self.log.append(("model.load_quantized_embedding_weights", a, {}))

    def calls(self, name):
        return [c for c in self.log if c[0] == name]


class _DenseHead:
    def __init__(self, log):
        self._log = log

    def load_shard_direct(self, *a):
        self._log.append(("lm_head.load_shard_direct", a, {}))


def _q(rng, out, inp, bits=4, g=64, scales_dtype=torch.float32):
    wq = torch.from_numpy(rng.integers(0, 2**32, (out, inp * bits // 32), dtype=np.uint64).astype(np.uint32))
    s = torch.from_numpy(rng.standard_normal((out, inp // g)).astype(np.float32)).to(scales_dtype)
    b = torch.from_numpy(rng.standard_normal((out, inp // g)).astype(np.float32)).to(scales_dtype)
    return wq, s, b


def _write(tmp_path, tensors, rank=0, mode=None):
    d = tmp_path / f"rank_{rank}"
    d.mkdir(parents=True, exist_ok=True)
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(d / "model.safetensors"))
    if mode is not None:
        (tmp_path / "config.json").write_text(json.dumps({"parallel": {"mode": mode}}))
    return tmp_path


def _llama_quantized(rng, L=2, D=128, I=256, V=96):
    t = {"model.embed_tokens.weight": torch.randn(V, D).to(torch.bfloat16),
         "model.norm.weight": torch.ones(D).to(torch.bfloat16)}
    for i in range(L):
        p = f"model.layers.{i}"
        t[f"{p}.input_layernorm.weight"] = torch.ones(D).to(torch.bfloat16)
        t[f"{p}.post_attention_layernorm.weight"] = torch.ones(D).to(torch.bfloat16)
        for name, (o, n) in {"self_attn.q_proj": (D, D), "self_attn.k_proj": (D // 2, D),
                             "self_attn.v_proj": (D // 2, D), "self_attn.o_proj": (D, D),
                             "mlp.gate_proj": (I, D), "mlp.up_proj": (I, D), "mlp.down_proj": (D, I)}.items():
            w, s, b = _q(rng, o, n)
            t[f"{p}.{name}.weight"], t[f"{p}.{name}.scales"], t[f"{p}.{name}.biases"] = w, s, b
    w, s, b = _q(rng, V, D, scales_dtype=torch.bfloat16)
    t["lm_head.weight"], t["lm_head.scales"], t["lm_head.biases"] = w, s, b
    return t


def test_quantized_llama_layout(tmp_path):
    rng = np.random.default_rng(0)
    t = _llama_quantized(rng)
    t["model.layers.1.self_attn.q_proj.bias"] = torch.zeros(128).to(torch.bfloat16)
    shard = _write(tmp_path, t, mode="tensor")
    assert ModelLoader.detect_quantization(shard) and detect_parallelism_mode(shard) == "tensor"
    m = FakeModel(2)
    asyncio.run(ModelLoader(0, 1, quantized=True).load_shards(m, shard))
    # dense vocab embedding (no embedding scales in the file)
    (name, a, _), = m.calls("embed_tokens.load_shard_direct")
    assert torch.equal(a[0], t["model.embed_tokens.weight"])
    for i in range(2):
        (_, _, kw), = m.calls(f"layers.{i}.attention.load_quantized_shards")
        p = f"model.layers.{i}.self_attn"
        for part, key in (("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "o_proj")):
            assert torch.equal(kw[f"{part}_weight"], t[f"{p}.{key}.weight"])
            assert kw[f"{part}_weight"].dtype == torch.uint32
            assert torch.equal(kw[f"{part}_scales"], t[f"{p}.{key}.scales"])
            assert torch.equal(kw[f"{part}_biases"], t[f"{p}.{key}.biases"])
        assert (kw["q_linear_bias"] is not None) == (i == 1) and kw["k_linear_bias"] is None
        (_, _, kw), = m.calls(f"layers.{i}.mlp.load_quantized_shards")
        p = f"model.layers.{i}.mlp"
        for part in ("gate", "up", "down"):
            assert torch.equal(kw[f"{part}_weight"], t[f"{p}.{part}_proj.weight"])
            assert torch.equal(kw[f"{part}_scales"], t[f"{p}.{part}_proj.scales"])
        assert len(m.calls(f"layers.{i}.input_layernorm.load_weights")) == 1
        assert len(m.calls(f"layers.{i}.post_attention_layernorm.load_weights")) == 1
    (_, a, _), = m.calls("norm.load_weights")
    assert torch.equal(a[0], t["model.norm.weight"]) and a[1] is None
    (_, a, _), = m.calls("lm_head.load_quantized_shard")
    assert torch.equal(a[0], t["lm_head.weight"]) and torch.equal(a[1], t["lm_head.scales"])
    # a loader constructed as unquantized takes the dense path (as the reference)
    m2 = FakeModel(2)
    asyncio.run(ModelLoader(0, 1, quantized=False).load_shards(m2, shard))
    assert m2.calls("layers.0.attention.load_shards") and not m2.calls("layers.0.attention.load_quantized_shards")


def test_phi2_names_and_shared_layernorm(tmp_path):
    D, I, V = 64, 128, 50
    t = {"model.embed_tokens.weight": torch.randn(V, D).to(torch.bfloat16),
         "model.final_layernorm.weight": torch.ones(D).to(torch.bfloat16),
         "model.final_layernorm.bias": torch.zeros(D).to(torch.bfloat16),
         "lm_head.weight": torch.randn(D, V).to(torch.bfloat16),
         "lm_head.bias": torch.zeros(V).to(torch.bfloat16)}
    p = "model.layers.0"
    t[f"{p}.input_layernorm.weight"] = torch.full((D,), 2.0).to(torch.bfloat16)
    t[f"{p}.input_layernorm.bias"] = torch.full((D,), 0.5).to(torch.bfloat16)
    for name in ("q_proj", "k_proj", "v_proj", "dense"):
        t[f"{p}.self_attn.{name}.weight"] = torch.randn(D, D).to(torch.bfloat16)
        t[f"{p}.self_attn.{name}.bias"] = torch.randn(D).to(torch.bfloat16)
    t[f"{p}.mlp.fc1.weight"] = torch.randn(D, I).to(torch.bfloat16)
    t[f"{p}.mlp.fc2.weight"] = torch.randn(I, D).to(torch.bfloat16)
    shard = _write(tmp_path, t)
    assert not ModelLoader.detect_quantization(shard) and detect_parallelism_mode(shard) == "tensor"
    m = FakeModel(1, lm_quantized=False)
    asyncio.run(ModelLoader(0, 1).load_shards(m, shard))
    (_, _, kw), = m.calls("layers.0.attention.load_shards")
    assert torch.equal(kw["o_weight"], t[f"{p}.self_attn.dense.weight"])
    assert torch.equal(kw["o_bias"], t[f"{p}.self_attn.dense.bias"])
    (_, _, kw), = m.calls("layers.0.mlp.load_shards")
    assert kw["gate_weight"] is None and torch.equal(kw["up_weight"], t[f"{p}.mlp.fc1.weight"])
    assert torch.equal(kw["down_weight"], t[f"{p}.mlp.fc2.weight"]) and kw["down_bias"] is None
    # no post-attention layernorm: the input layernorm's weight and bias serve both
    (_, a, _), = m.calls("layers.0.post_attention_layernorm.load_weights")
    assert torch.equal(a[0], t[f"{p}.input_layernorm.weight"]) and torch.equal(a[1], t[f"{p}.input_layernorm.bias"])
    (_, a, _), = m.calls("norm.load_weights")
    assert torch.equal(a[1], t["model.final_layernorm.bias"])
    (_, a, _), = m.calls("lm_head.load_shard_direct")
    assert torch.equal(a[0], t["lm_head.weight"]) and torch.equal(a[1], t["lm_head.bias"])


def test_quantized_embedding_and_bf16_bit_patterns(tmp_path):
    rng = np.random.default_rng(1)
    D, V = 128, 40
    w, s, b = _q(rng, V, D)
    norm_bits = torch.from_numpy(np.full(D, 0x3F80, np.uint16))      # bf16 1.0 stored as u16
    t = {"model.embed_tokens.weight": w, "model.embed_tokens.scales": s, "model.embed_tokens.biases": b,
         "model.norm.weight": norm_bits}
    shard = _write(tmp_path, t, mode="pipeline")
    assert detect_parallelism_mode(shard) == "pipeline"
    m = FakeModel(0)
    asyncio.run(ModelLoader(0, 1, quantized=True).load_shards(m, shard))
    (_, a, _), = m.calls("model.load_quantized_embedding_weights")
    assert torch.equal(a[0], w) and torch.equal(a[1], s) and torch.equal(a[2], b)
    (_, a, _), = m.calls("norm.load_weights")
    assert a[0].dtype == torch.bfloat16 and torch.equal(a[0].float(), torch.ones(D))


def test_missing_rank_and_absent_files(tmp_path):
    assert detect_parallelism_mode(tmp_path) == "tensor"
    assert not ModelLoader.detect_quantization(tmp_path, rank=3)
    with pytest.raises(FileNotFoundError, match="rank_1"):
        asyncio.run(ModelLoader(1, 2).load_shards(FakeModel(0), tmp_path))
