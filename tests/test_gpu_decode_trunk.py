"""The whole-trunk batch-1 decode launch against the per-op decode path.

Both paths run the same quantized model from the same prefilled cache, one token
at a time, with the same input token each step (teacher forcing).  Checks:

* the first layer's appended key and value are bit-identical (embedding, fused
  RMSNorm, q|k|v product and rotation share the per-op kernels' arithmetic);
* logits of every step within LOGIT_TOL max-abs-rel (attention rounds
  differently: fp32 probabilities instead of bf16);
* every layer's cache within LOGIT_TOL;
* graph replay of the fused step equals its eager run bit for bit;
* the plan's status word stays 0 (no launch gave up waiting).

Shapes: a GQA model with head_dim 128 and 4 query heads per kv head (the
Llama-3-8B geometry), W4 and W8, and two Llama-3-8B-shape layers.
"""
import asyncio

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32
from shardcompute_amd import _lib
from shardcompute_amd.decode_plan import TrunkPlan, eligible
from shardcompute_amd.executor import DecodeGraph
from shardcompute_amd.parallel.transformer import ParallelTransformer
from tests.gpu_util import host_u16

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2

SMALL = dict(hidden=2048, inter=2048, heads=16, kv_heads=4, vocab=2048, layers=3)
LLAMA8B_2L = dict(hidden=4096, inter=14336, heads=32, kv_heads=8, vocab=4096, layers=2)


def build(cfg, bits, capacity, seed=0):
    dev = torch.device("cuda", 0)
    H, I, V = cfg["hidden"], cfg["inter"], cfg["vocab"]
    D = H // cfg["heads"]
    nq, nkv = cfg["heads"] * D, cfg["kv_heads"] * D
    m = ParallelTransformer(vocab_size=V, hidden_size=H, num_layers=cfg["layers"], num_heads=cfg["heads"],
                            intermediate_size=I, world_size=1, rank=0, num_kv_heads=cfg["kv_heads"],
                            max_position_embeddings=capacity, rms_norm_eps=1e-5, rope_base=500000.0,
                            use_quantized=True, quantization_bits=bits, quantization_group_size=64,
                            embedding="vocab", quantized_lm_head=True, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def q(n, k):
        return _lib.quantize(torch.randn((n, k), generator=g, device=dev).mul_(0.02), bits=bits)

    def norm_w():
        return (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)

    for layer in m.layers:
        layer.input_layernorm.load_weights(norm_w())
        layer.post_attention_layernorm.load_weights(norm_w())
        wq, s, b = q(nq + 2 * nkv, H)
        sl = [slice(0, nq), slice(nq, nq + nkv), slice(nq + nkv, nq + 2 * nkv)]
        layer.attention.load_quantized_shards(wq[sl[0]], s[sl[0]], b[sl[0]], None, wq[sl[1]], s[sl[1]], b[sl[1]],
                                              None, wq[sl[2]], s[sl[2]], b[sl[2]], None, *q(H, nq), None)
        gwq, gs, gb = q(2 * I, H)
        layer.mlp.load_quantized_shards(gwq[I:], gs[I:], gb[I:], None, *q(H, I), None, gwq[:I], gs[:I], gb[:I],
                                        None)
    m.load_embedding_weights(torch.randn((V, H), generator=g, device=dev).mul_(0.02).to(torch.bfloat16))
    m.load_norm_weights(norm_w())
    m.load_quantized_lm_head_weights(*q(V, H))
    torch.cuda.synchronize()
    return m


def f32(t):
    return bf16_to_f32(host_u16(t.reshape(-1)))


def rel(a, b):
    a, b = f32(a).astype(np.float64), f32(b).astype(np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def clone_cache(model, c):
    d = model.new_cache(c.batch, c.capacity)
    d.k.copy_(c.k)
    d.vt.copy_(c.vt)
    d.counters.copy_(c.counters)
    d.length = c.length
    return d


def compare_paths(model, prompt_len, steps, capacity, seed=1, tol=LOGIT_TOL):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    ids = torch.randint(0, model.vocab_size, (1, prompt_len), generator=gen, device="cuda")
    ca = model.new_cache(1, capacity)
    logits, _ = asyncio.run(model.forward(ids, past_key_values=ca, use_cache=True, last_only=True))
    cb = clone_cache(model, ca)
    tok_a = torch.zeros((1, steps + 2), dtype=torch.int32, device="cuda")
    tok_b = torch.zeros_like(tok_a)
    da = DecodeGraph(model, ca, tok_a, use_graph=False, fused_trunk=False)
    db = DecodeGraph(model, cb, tok_b, use_graph=False, fused_trunk=True)
    assert da.bufs.plan is None and db.bufs.plan is not None
    for d, c, t in ((da, ca, tok_a), (db, cb, tok_b)):
        _lib.argmax(logits.reshape(1, -1), ids=d.bufs.ids.view(-1), tokens=t, step=c.counters[1:])
        _lib.add_i32(c.counters[1:], 1, n=1)
    worst = 0.0
    for s in range(steps):
        pos = ca.length
        db.bufs.ids.copy_(da.bufs.ids)          # teacher forcing: the same input token
        da.run(1)
        db.run(1)
        torch.cuda.synchronize()
        assert db.bufs.plan.status() == 0, f"trunk launch gave up at step {s}"
        # layer 0's appended key/value: bit-identical
        assert torch.equal(ca.k[0][:, :, pos], cb.k[0][:, :, pos]), f"layer-0 key differs at step {s}"
        assert torch.equal(ca.vt[0][..., pos], cb.vt[0][..., pos]), f"layer-0 value differs at step {s}"
        r = rel(db.logits, da.logits)
        worst = max(worst, r)
        assert r <= tol, f"step {s} (position {pos}): logits max-abs-rel {r:.3e}"
    n = ca.length
    for i in range(len(model.layers)):
        assert rel(cb.k[i][:, :, :n], ca.k[i][:, :, :n]) <= tol, f"layer {i} keys"
        assert rel(cb.vt[i][..., :n], ca.vt[i][..., :n]) <= tol, f"layer {i} values"
    return worst


@pytest.fixture(scope="module")
def small_w4():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return build(SMALL, 4, 512)


def test_eligibility(small_w4):
    m = small_w4
    c = m.new_cache(1, 64)
    assert eligible(m, c) == (True, "")
    assert eligible(m, m.new_cache(2, 64))[0] is False


TINY = dict(hidden=2048, inter=5632, heads=32, kv_heads=4, vocab=2048, layers=3)


@pytest.fixture(scope="module")
def tiny_w4():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return build(TINY, 4, 512, seed=7)


@pytest.mark.parametrize("prompt_len", [1, 37, 300])
def test_trunk_matches_per_op_tinyllama_heads(tiny_w4, prompt_len):
    # head_dim 64, 8 query heads per kv head; layers under 32 MB run on one workgroup
    # per two CUs (32 key ranges per kv head on 256 CUs)
    assert eligible(tiny_w4, tiny_w4.new_cache(1, 64)) == (True, "")
    print(f"trunk vs per-op: W4 TinyLlama heads, prompt {prompt_len}", flush=True)
    worst = compare_paths(tiny_w4, prompt_len, steps=6, capacity=512)
    print(f"  worst logits max-abs-rel {worst:.2e}", flush=True)


@pytest.mark.parametrize("prompt_len", [1, 37, 300])
def test_trunk_matches_per_op_w4(small_w4, prompt_len):
    print(f"trunk vs per-op: W4 small, prompt {prompt_len}", flush=True)
    worst = compare_paths(small_w4, prompt_len, steps=6, capacity=512)
    print(f"  worst logits max-abs-rel {worst:.2e}", flush=True)


def test_trunk_graph_replay_equals_eager(small_w4):
    m = small_w4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    ids = torch.randint(0, m.vocab_size, (1, 20), generator=gen, device="cuda")
    ca = m.new_cache(1, 128)
    logits, _ = asyncio.run(m.forward(ids, past_key_values=ca, use_cache=True, last_only=True))
    cb = clone_cache(m, ca)
    outs = []
    for c, use_graph in ((ca, False), (cb, True)):
        t = torch.zeros((1, 16), dtype=torch.int32, device="cuda")
        d = DecodeGraph(m, c, t, use_graph=use_graph, fused_trunk=True)
        _lib.argmax(logits.reshape(1, -1), ids=d.bufs.ids.view(-1), tokens=t, step=c.counters[1:])
        _lib.add_i32(c.counters[1:], 1, n=1)
        for _ in range(5):
            d.run(1)
            torch.cuda.synchronize()      # eager work between replays
        assert d.bufs.plan.status() == 0
        outs.append((t.clone(), c.k.clone(), c.vt.clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][2], outs[1][2])


@pytest.mark.parametrize("fused", [True, False])
def test_multi_step_graph_equals_eager(small_w4, fused):
    # 13 steps: one eager step, then replays of a 4-step graph (run(4), run(8)) mixed
    # with single-step replays (run(3), the tail), with eager work in between
    m = small_w4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    ids = torch.randint(0, m.vocab_size, (1, 30), generator=gen, device="cuda")
    ca = m.new_cache(1, 128)
    logits, _ = asyncio.run(m.forward(ids, past_key_values=ca, use_cache=True, last_only=True))
    cb = clone_cache(m, ca)
    outs = []
    for c, use_graph in ((ca, False), (cb, True)):
        print(f"multi-step graph: fused trunk {fused}, graphs {use_graph}", flush=True)
        t = torch.zeros((1, 16), dtype=torch.int32, device="cuda")
        d = DecodeGraph(m, c, t, use_graph=use_graph, fused_trunk=fused, steps_per_graph=4)
        _lib.argmax(logits.reshape(1, -1), ids=d.bufs.ids.view(-1), tokens=t, step=c.counters[1:])
        _lib.add_i32(c.counters[1:], 1, n=1)
        for n in (1, 4, 3, 8, 1):
            d.run(n)
            torch.cuda.synchronize()
        assert c.length == 30 + 17 and c.counters[:2].tolist() == [47, 18]
        assert d.bufs.plan is None or d.bufs.plan.status() == 0
        outs.append((t.clone(), c.k.clone(), c.vt.clone(), d.logits.clone()))
    assert use_graph and cb.length == ca.length
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)


WIDE_SMALL = dict(hidden=4096, inter=1024, heads=32, kv_heads=8, vocab=2048, layers=2)


@pytest.mark.parametrize("prompt_len", [5, 300])
def test_trunk_matches_per_op_two_merge_batches(prompt_len):
    # 27 MB layers run on half the CUs: 4096 attention outputs over 128 workgroups is
    # 32 values per merging workgroup, merged and published in two batches of 16
    m = build(WIDE_SMALL, 4, 512, seed=11)
    assert eligible(m, m.new_cache(1, 64)) == (True, "")
    print(f"trunk vs per-op: 32 values per merging workgroup, prompt {prompt_len}", flush=True)
    worst = compare_paths(m, prompt_len, steps=4, capacity=512)
    print(f"  worst logits max-abs-rel {worst:.2e}", flush=True)


def test_trunk_matches_per_op_w8():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    print("trunk vs per-op: W8 small, prompt 50", flush=True)
    m = build(SMALL, 8, 256, seed=5)
    compare_paths(m, 50, steps=4, capacity=256)


def test_trunk_matches_per_op_llama3_8b_shape():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    print("trunk vs per-op: Llama-3-8B shape, 2 layers, prompt 130", flush=True)
    m = build(LLAMA8B_2L, 4, 256, seed=7)
    compare_paths(m, 130, steps=4, capacity=256)


def test_trunk_matches_per_op_long_context():
    """Keys per attention unit > 8: every unit's keys span several items, which the
    worker waves take in claim order; the item states merge in item order."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    print("trunk vs per-op: Llama-3-8B shape, 2 layers, prompt 900", flush=True)
    m = build(LLAMA8B_2L, 4, 1024, seed=9)
    worst = compare_paths(m, 900, steps=3, capacity=1024)
    print(f"  worst logits max-abs-rel {worst:.2e}", flush=True)


def test_control_wave_item_same_bits(monkeypatch):
    """2049-2304 positions on the Llama-3-8B shape (32 key ranges per kv head): 9
    items per attention unit for 8 worker waves, so the control wave computes each
    unit's last item from its own LDS area (loaded while q|k|v is computed).  The
    item states merge in item order, so the steps are bit for bit those of a plan in
    which the workers take every item (SC_TRUNK_CONTROL_ITEM=0 at plan creation), and
    within the tolerance of the per-op path."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    m = build(LLAMA8B_2L, 4, 2304, seed=13)
    print("trunk control-wave item: Llama-3-8B shape, 2 layers, prompt 2060 vs per-op", flush=True)
    worst = compare_paths(m, 2060, steps=3, capacity=2304)
    print(f"  worst logits max-abs-rel {worst:.2e}", flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(6)
    ids = torch.randint(0, m.vocab_size, (1, 2060), generator=gen, device="cuda")
    ca = m.new_cache(1, 2304)
    logits, _ = asyncio.run(m.forward(ids, past_key_values=ca, use_cache=True, last_only=True))
    cb = clone_cache(m, ca)
    outs = []
    for c, env in ((ca, None), (cb, "0")):
        print(f"trunk control-wave item: SC_TRUNK_CONTROL_ITEM={env}", flush=True)
        if env is None:
            monkeypatch.delenv("SC_TRUNK_CONTROL_ITEM", raising=False)
        else:
            monkeypatch.setenv("SC_TRUNK_CONTROL_ITEM", env)
        t = torch.zeros((1, 8), dtype=torch.int32, device="cuda")
        d = DecodeGraph(m, c, t, use_graph=False, fused_trunk=True)
        assert d.bufs.plan is not None
        _lib.argmax(logits.reshape(1, -1), ids=d.bufs.ids.view(-1), tokens=t, step=c.counters[1:])
        _lib.add_i32(c.counters[1:], 1, n=1)
        d.run(5)
        torch.cuda.synchronize()
        assert d.bufs.plan.status() == 0
        outs.append((t.clone(), c.k.clone(), c.vt.clone(), d.logits.clone()))
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)


def test_trunk_repeatable_long_context():
    """Two fused runs from the same cache give bit-identical caches and tokens, also
    when the attention items of a unit land on different waves from run to run."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    m = build(SMALL, 4, 1536, seed=11)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    ids = torch.randint(0, m.vocab_size, (1, 1300), generator=gen, device="cuda")
    ca = m.new_cache(1, 1536)
    logits, _ = asyncio.run(m.forward(ids, past_key_values=ca, use_cache=True, last_only=True))
    cb = clone_cache(m, ca)
    outs = []
    for c in (ca, cb):
        t = torch.zeros((1, 8), dtype=torch.int32, device="cuda")
        d = DecodeGraph(m, c, t, use_graph=False, fused_trunk=True)
        _lib.argmax(logits.reshape(1, -1), ids=d.bufs.ids.view(-1), tokens=t, step=c.counters[1:])
        _lib.add_i32(c.counters[1:], 1, n=1)
        d.run(4)
        torch.cuda.synchronize()
        assert d.bufs.plan.status() == 0
        outs.append((t.clone(), c.k.clone(), c.vt.clone(), d.logits.clone()))
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)


def test_plan_rejects_unsupported_shapes():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    # 8 query heads per kv head: the per-op path runs
    cfg = dict(hidden=1024, inter=1024, heads=8, kv_heads=1, vocab=512, layers=1)
    m = build(cfg, 4, 64)
    c = m.new_cache(1, 64)
    assert eligible(m, c)[0] is False
    with pytest.raises(ValueError):
        TrunkPlan(m, c, torch.zeros(1, dtype=torch.int32, device="cuda"),
                  torch.zeros(1024, dtype=torch.bfloat16, device="cuda"))


def test_trunk_op_timeline(small_w4):
    """The plan's op timeline: with tracing on, every workgroup stamps every op in
    order (items computed <= published, input polled <= staged, staged before the
    op's items are computed), the outputs equal an untraced launch's, and the
    per-op-kind summary spans the launch."""
    m = small_w4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(6)
    ids = torch.randint(0, m.vocab_size, (1, 40), generator=gen, device="cuda")
    ca = m.new_cache(1, 128)
    logits, _ = asyncio.run(m.forward(ids, past_key_values=ca, use_cache=True, last_only=True))
    cb = clone_cache(m, ca)
    outs = []
    for c, traced in ((ca, False), (cb, True)):
        t = torch.zeros((1, 8), dtype=torch.int32, device="cuda")
        d = DecodeGraph(m, c, t, use_graph=False, fused_trunk=True)
        if traced:
            d.bufs.plan.trace(True)
        _lib.argmax(logits.reshape(1, -1), ids=d.bufs.ids.view(-1), tokens=t, step=c.counters[1:])
        _lib.add_i32(c.counters[1:], 1, n=1)
        d.run(2)
        torch.cuda.synchronize()
        assert d.bufs.plan.status() == 0
        outs.append((t.clone(), c.k.clone(), c.vt.clone()))
        if traced:
            st = d.bufs.plan.read_trace()
            P, nops, _ = st.shape
            # one workgroup per CU, or per two CUs for layers under 32 MB of weights
            cus = torch.cuda.get_device_properties(0).multi_processor_count
            assert nops == 1 + 6 * len(m.layers) and P in (cus, cus // 2)
            comp, pub, pol, stg = st[..., 0], st[..., 1], st[..., 2], st[..., 3]
            assert (pub >= comp).all() and (stg >= pol).all() and (comp >= stg).all()
            assert (pol[:, 1:] >= pub[:, :-1]).all()
            tl = d.bufs.plan.timeline()
            assert set(tl["ops"]) == set(TrunkPlan.OP_KINDS) and tl["per_layer_us"] > 0
            d.bufs.plan.trace(False)
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)
