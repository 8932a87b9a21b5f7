"""The decoder stack on the GPU against the oracle's restatement, same packed weights.

A 3-layer GQA decoder (vocab 1000, hidden 512, 8 q / 2 kv heads of 64,
intermediate 1536, W4 g64, bf16 vocab embedding, W4 lm_head) exercises every
kernel on the path.  Checks:

* prefill logits (all positions, batch 1 and 2) within LOGIT_TOL max-abs-rel;
* greedy generation: each GPU token is the oracle's argmax up to a small margin
  (the oracle teacher-forced with the GPU's tokens, step by step);
* graph-replayed decode against eager decode, the incremental KV-cache path
  against one full forward, and the reference-layout tuple cache against the
  preallocated cache;
* the block- and attention-level APIs against the oracle's single layer.
"""
import asyncio

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16, round_bf16
from oracle.decoder import DecoderShape, OracleDecoder, random_decoder_weights, rms_norm
from shardcompute_amd.executor import ParallelExecutor
from shardcompute_amd.kv_cache import KVCache
from shardcompute_amd.parallel.transformer import ParallelTransformer
from tests.gpu_util import dev, dev_bf16, host_u16

pytestmark = pytest.mark.gpu

LOGIT_TOL = 3e-2
SHAPE = DecoderShape(vocab_size=1000, hidden_size=512, num_layers=3, num_heads=8, num_kv_heads=2,
                     intermediate_size=1536, rope_theta=10000.0)


@pytest.fixture(scope="module")
def weights():
    return random_decoder_weights(SHAPE, seed=0)


def build_model(shape, W, max_pos=256):
    m = ParallelTransformer(vocab_size=shape.vocab_size, hidden_size=shape.hidden_size,
                            num_layers=shape.num_layers, num_heads=shape.num_heads,
                            intermediate_size=shape.intermediate_size, world_size=1, rank=0,
                            num_kv_heads=shape.num_kv_heads, max_position_embeddings=max_pos,
                            rms_norm_eps=shape.rms_norm_eps, rope_base=shape.rope_theta, use_quantized=True,
                            quantization_bits=shape.bits, quantization_group_size=shape.group_size,
                            embedding="vocab", quantized_lm_head=True)
    m.load_embedding_weights(W["embed"])
    for layer, L in zip(m.layers, W["layers"]):
        layer.input_layernorm.load_weights(L["input_ln"])
        layer.post_attention_layernorm.load_weights(L["post_ln"])
        q, k, v, o = L["q"], L["k"], L["v"], L["o"]
        layer.attention.load_quantized_shards(q.wq, q.scales, q.biases, None, k.wq, k.scales, k.biases, None,
                                              v.wq, v.scales, v.biases, None, o.wq, o.scales, o.biases, None)
        g, u, d = L["gate"], L["up"], L["down"]
        layer.mlp.load_quantized_shards(u.wq, u.scales, u.biases, None, d.wq, d.scales, d.biases, None,
                                        g.wq, g.scales, g.biases, None)
    m.load_norm_weights(W["norm"])
    lm = W["lm_head"]
    m.load_quantized_lm_head_weights(lm.wq, lm.scales, lm.biases)
    return m


@pytest.fixture(scope="module")
def model(weights):
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return build_model(SHAPE, weights)


def run(coro):
    return asyncio.run(coro)


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def logits_np(t):
    return bf16_to_f32(host_u16(t.reshape(-1, t.shape[-1]))).reshape(t.shape)


@pytest.mark.parametrize("B,S", [(1, 24), (2, 9)])
def test_prefill_logits(device, weights, model, B, S):
    ids = np.random.default_rng(S).integers(0, SHAPE.vocab_size, (B, S))
    got, _ = run(model.forward(dev(ids.astype(np.int32))))
    ref = OracleDecoder(SHAPE, weights).forward(ids)
    err = rel(logits_np(got), ref)
    print(f"prefill B={B} S={S}: logits max-abs-rel {err:.2e}", flush=True)
    assert got.shape == (B, S, SHAPE.vocab_size)
    assert err <= LOGIT_TOL


def _margin_check(gpu_new, steps, margin_frac=0.02):
    agree = 0
    for t, lg in enumerate(steps):
        for b in range(lg.shape[0]):
            tok = int(gpu_new[b, t])
            top = lg[b].max()
            assert lg[b, tok] >= top - margin_frac * np.abs(lg[b]).max(), (t, b, tok, lg[b, tok], top)
            agree += int(tok == int(np.argmax(lg[b])))
    return agree / (len(steps) * steps[0].shape[0])


@pytest.mark.parametrize("B,use_graphs", [(1, True), (2, True), (1, False)])
def test_greedy_generation(device, weights, model, B, use_graphs):
    S, n = 17, 20
    ids = np.random.default_rng(100 + B).integers(0, SHAPE.vocab_size, (B, S))
    ex = ParallelExecutor(0, 1, None, model, use_graphs=use_graphs)
    out = run(ex.generate(dev(ids.astype(np.int64)), max_new_tokens=n, temperature=0.0))
    out = out.cpu().numpy()
    assert out.shape == (B, S + n) and np.array_equal(out[:, :S], ids)
    new = out[:, S:]
    _, steps = OracleDecoder(SHAPE, weights).generate_greedy(ids, n, forced=new)
    agree = _margin_check(new, steps)
    print(f"greedy B={B} graphs={use_graphs}: argmax agreement {agree:.2f}", flush=True)
    # every token passed the margin check; exact argmax agreement measured 0.95-1.00
    # (the misses are near-ties of the random-init logits)
    assert agree >= 0.9


def test_graph_matches_eager(device, model):
    ids = np.random.default_rng(5).integers(0, SHAPE.vocab_size, (1, 12)).astype(np.int64)
    outs = []
    for g in (False, True):
        ex = ParallelExecutor(0, 1, None, model, use_graphs=g)
        outs.append(run(ex.generate(dev(ids), max_new_tokens=16, temperature=0.0)).cpu().numpy())
    # the kernels are the same; split-tile sums may add in another order, so allow a
    # late divergence only
    same = int(np.argmax(outs[0] != outs[1])) if (outs[0] != outs[1]).any() else outs[0].shape[1]
    assert same >= 12 + 12


def test_stop_tokens_and_callback(device, model):
    ids = np.random.default_rng(6).integers(0, SHAPE.vocab_size, (1, 10)).astype(np.int64)
    ex = ParallelExecutor(0, 1, None, model, check_every=4)
    full = run(ex.generate(dev(ids), max_new_tokens=12, temperature=0.0)).cpu().numpy()[0, 10:]
    stop_at = 5
    seen = []

    async def cb(tok, idx, last):
        seen.append((tok, idx, last))

    out = run(ex.generate(dev(ids), max_new_tokens=12, temperature=0.0, stop_tokens=[int(full[stop_at])],
                          token_callback=cb)).cpu().numpy()[0, 10:]
    first = int(np.argmax(full == full[stop_at]))
    assert np.array_equal(out, full[:first + 1])
    assert [s[0] for s in seen] == list(out) and seen[-1][2] and not any(s[2] for s in seen[:-1])


def test_incremental_matches_full_forward(device, model):
    ids = np.random.default_rng(9).integers(0, SHAPE.vocab_size, (1, 20)).astype(np.int32)
    full, _ = run(model.forward(dev(ids)))
    cache = model.new_cache(1, 64)
    l0, _ = run(model.forward(dev(ids[:, :16]), past_key_values=cache, use_cache=True))
    steps = [l0[:, -1]]
    for t in range(16, 20):
        lt, _ = run(model.forward(dev(ids[:, t:t + 1]), past_key_values=cache, use_cache=True))
        steps.append(lt[:, -1])
    fl = logits_np(full)[0]
    for i, lt in enumerate(steps[:-1]):
        assert rel(logits_np(lt)[0], fl[15 + i]) <= LOGIT_TOL
    assert cache.length == 20


def test_tuple_cache_matches_preallocated(device, model):
    ids = np.random.default_rng(10).integers(0, SHAPE.vocab_size, (1, 14)).astype(np.int32)
    la, past = run(model.forward(dev(ids[:, :10]), use_cache=True))
    assert isinstance(past, list) and past[0][0].shape == (1, SHAPE.num_kv_heads, 10, SHAPE.head_dim)
    lb, past2 = run(model.forward(dev(ids[:, 10:]), past_key_values=past, use_cache=True))
    assert past2[0][0].shape[2] == 14
    cache = model.new_cache(1, 32)
    run(model.forward(dev(ids[:, :10]), past_key_values=cache, use_cache=True))
    lc, _ = run(model.forward(dev(ids[:, 10:]), past_key_values=cache, use_cache=True))
    assert rel(logits_np(lb), logits_np(lc)) <= 1e-2
    kk, vv = cache.as_tuples()[1]
    assert torch.equal(kk, past2[1][0]) and torch.equal(vv, past2[1][1])


def test_block_api_matches_oracle(device, weights, model):
    rng = np.random.default_rng(12)
    x = f32_to_bf16(rng.standard_normal((1, 6, SHAPE.hidden_size)).astype(np.float32))
    h, cache = run(model.layers[0].forward(dev_bf16(x), use_cache=True))
    o = OracleDecoder(SHAPE, weights)
    L = weights["layers"][0]
    x32 = bf16_to_f32(x)
    xn = rms_norm(x32, L["input_ln"], SHAPE.rms_norm_eps)
    hr = round_bf16(x32 + o._attn(0, xn, L))
    xn = rms_norm(hr, L["post_ln"], SHAPE.rms_norm_eps)
    hr = round_bf16(hr + o._mlp(xn, L))
    assert rel(bf16_to_f32(host_u16(h)), hr) <= LOGIT_TOL
    assert cache[0].shape == (1, SHAPE.num_kv_heads, 6, SHAPE.head_dim)


def test_prefill_with_additive_mask(device, weights, model):
    # the reference's attention_mask, added by every layer to its scaled scores
    # (transformer.py:548-553, attention.py:449-450), against the oracle
    rng = np.random.default_rng(21)
    B, S = 2, 9
    ids = rng.integers(0, SHAPE.vocab_size, (B, S))
    m = (rng.standard_normal((B, 1, S, S)) * 2).astype(np.float32)
    m[0, 0, :, 3] = -np.inf
    m[1, 0, 5:, 1:4] = -np.inf
    logits, _ = run(model.forward(torch.from_numpy(ids).cuda(), attention_mask=torch.from_numpy(m).cuda()))
    ref = OracleDecoder(SHAPE, weights).forward(ids, mask=m)
    assert rel(logits_np(logits), ref) <= LOGIT_TOL
    # a zero mask (the masked kernel) equals no mask
    z, _ = run(model.forward(torch.from_numpy(ids).cuda(), attention_mask=torch.zeros((1, 1, 1, S), device="cuda")))
    plain, _ = run(model.forward(torch.from_numpy(ids).cuda()))
    assert rel(logits_np(z), logits_np(plain)) <= 1e-2


def test_attention_forward_sync_partial(device, weights, model):
    # cache-less attention rotated for positions offset..offset+S-1 equals the cached
    # path when the cache starts at that offset with no earlier keys visible only if
    # offset == 0; check the offset-0 case against forward() and the rotation shift
    # through the RoPE object
    att = model.layers[1].attention
    rng = np.random.default_rng(13)
    x = dev_bf16(f32_to_bf16(rng.standard_normal((1, 5, SHAPE.hidden_size)).astype(np.float32)))
    a = att.forward_sync_partial(x, position_offset=0)
    b, _ = run(att.forward(x))
    assert torch.equal(a, b)
    q = dev_bf16(f32_to_bf16(rng.standard_normal((1, 8, 5, 64)).astype(np.float32)))
    k = dev_bf16(f32_to_bf16(rng.standard_normal((1, 2, 5, 64)).astype(np.float32)))
    q1, k1 = att.rope(q, k, position_offset=7)
    from oracle.decoder import apply_rope, rope_cos_sin
    cos, sin = rope_cos_sin(np.arange(7, 12), 64, SHAPE.rope_theta)
    assert np.array_equal(host_u16(q1), f32_to_bf16(apply_rope(bf16_to_f32(host_u16(q)), cos, sin)))
    assert np.array_equal(host_u16(k1), f32_to_bf16(apply_rope(bf16_to_f32(host_u16(k)), cos, sin)))


def test_model_loader_roundtrip(device, weights, model, tmp_path):
    # the same packed weights written as the reference's rank_0/model.safetensors
    # (Hugging Face names, fp32 scales/biases as the reference's quantizer leaves
    # them) and loaded through ModelLoader give bit-identical logits
    from safetensors.torch import save_file
    from shardcompute_amd.loader import ModelLoader

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)

    def u32(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).view(torch.uint32)

    W = weights
    t = {"model.embed_tokens.weight": bf(W["embed"]), "model.norm.weight": bf(W["norm"])}
    for i, L in enumerate(W["layers"]):
        p = f"model.layers.{i}"
        t[f"{p}.input_layernorm.weight"] = bf(L["input_ln"])
        t[f"{p}.post_attention_layernorm.weight"] = bf(L["post_ln"])
        for key, name in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                          ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                          ("down", "mlp.down_proj")):
            q = L[key]
            t[f"{p}.{name}.weight"] = u32(q.wq)
            t[f"{p}.{name}.scales"] = bf(q.scales).float()
            t[f"{p}.{name}.biases"] = bf(q.biases).float()
    lm = W["lm_head"]
    t["lm_head.weight"], t["lm_head.scales"], t["lm_head.biases"] = u32(lm.wq), bf(lm.scales), bf(lm.biases)
    (tmp_path / "rank_0").mkdir()
    save_file(t, str(tmp_path / "rank_0" / "model.safetensors"))

    assert ModelLoader.detect_quantization(tmp_path)
    m2 = ParallelTransformer(vocab_size=SHAPE.vocab_size, hidden_size=SHAPE.hidden_size,
                             num_layers=SHAPE.num_layers, num_heads=SHAPE.num_heads,
                             intermediate_size=SHAPE.intermediate_size, world_size=1, rank=0,
                             num_kv_heads=SHAPE.num_kv_heads, max_position_embeddings=256,
                             rms_norm_eps=SHAPE.rms_norm_eps, rope_base=SHAPE.rope_theta, use_quantized=True,
                             quantization_bits=SHAPE.bits, quantization_group_size=SHAPE.group_size,
                             embedding="vocab", quantized_lm_head=True)
    run(ModelLoader(0, 1, quantized=True).load_shards(m2, tmp_path))
    ids = dev(np.random.default_rng(21).integers(0, SHAPE.vocab_size, (2, 9)).astype(np.int64))
    a, _ = run(model.forward(ids))
    b, _ = run(m2.forward(ids))
    torch.cuda.synchronize()
    assert torch.equal(a, b)
