"""The decoder configurations at their stated workloads, end to end on one GPU.

* TinyLlama-1.1B shape (22 layers, hidden 2048, intermediate 5632, 32 q / 4 kv
  heads of 64, vocab 32000, RoPE theta 10000), W4 g64, bf16 embedding: greedy
  decode of 128 tokens from one 32-token uniform-random prompt (numpy seed 0)
  through ``ParallelExecutor.generate``, against the oracle decoder
  teacher-forced with the GPU's tokens: every step's logits within DEEP_LOGIT_TOL,
  every token within a 2 % margin of the oracle's maximum (so every step whose
  oracle top-2 gap exceeds that margin has the oracle's token exactly; closer
  steps are near-ties of the random-init logits and are only reported).
* Llama-3-8B shape (32 layers), 2048-token prefill, properties at full size:
  the whole-trunk decode against the per-op decode for all 256 decode steps of
  the workload (teacher-forced, positions 2048-2303); batch 16 of 16 prompts for
  256 steps, three of its rows against batch-1 decode of their prompts at the
  last positions;
  batch 16 with 16 copies of one prompt gives 16 bit-identical rows, whose
  logits match batch-1 decode of that prompt; the prefill's last-position
  logits match prefilling all but the last token and decoding it.
* Llama-3-70B rank-0 shard of world_size 8 (80 layers, hidden 8192, 8 q / 1 kv
  head of 128, intermediate 3584 per rank, the all-reduces as identity), W4 and
  W8: layer 0 of the shard against the oracle on the same packed weights;
  batch-32 decode of the workload's 128 tokens after a 1024-token prefill, finite
  at every step, whose row 5 matches batch-1 decode of that prompt (teacher-forced)
  at the last 8 positions.
"""
import asyncio

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32
from oracle.decoder import DecoderShape, OracleDecoder, QLinear, rms_norm
from shardcompute_amd import _lib
from shardcompute_amd.communicator import IdentityCommunicator
from shardcompute_amd.executor import DecodeGraph, ParallelExecutor
from shardcompute_amd.parallel.transformer import ParallelTransformer
from tests.gpu_util import host_u16, host_u32
from tests.test_gpu_trunk_oracle import gpu_model_and_oracle

pytestmark = pytest.mark.gpu

LOGIT_TOL = 3e-2
# Deep models amplify the per-op bf16 roundings (each op rounds its output once;
# two implementations, or two kernel paths, sum in different orders) through the
# residual stream of random-init layers.  Measured: TinyLlama (22 layers) against
# the oracle 0.019-0.033 over 128 steps; Llama-3-8B (32 layers) between kernel
# paths 0.043-0.063; the 70B shard (80 layers) 0.061-0.064, while its layer 0 is
# within 0.0095 of the oracle.  A wiring or indexing error gives O(1) differences.
DEEP_LOGIT_TOL = 6e-2        # 22 layers, against the oracle
PATH_TOL_32 = 8e-2           # 32 layers, between kernel paths
# 80 layers, batch 32 against batch 1 (the 32-row kernels against the batch-1 GEMV at
# every projection, the attention split differently, and the prefill's q|k|v at
# 1024 rows with K split against whole K at 32768): measured over 128 decode steps at
# positions 1024-1151, W4 and W8, max-abs-rel 0.07-0.11 and rms-relative 0.07-0.11,
# flat in the position (no growth from step 1 to step 127).  The floor is set by the
# depth: the prefill's logits alone (step 0) move by 0.087 rms-relative when only the
# order of layer 0's q|k|v fp32 sums changes (K split in two at 1024 rows).
PATH_TOL_80 = 1.5e-1
PATH_RMS_80 = 1.5e-1

def run(coro):
    return asyncio.run(coro)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / np.abs(b).max())


def f32(t):
    return bf16_to_f32(host_u16(t.reshape(-1, t.shape[-1])))


# ---------------------------------------------------------------- TinyLlama, 22 layers

TINYLLAMA = dict(hidden=2048, inter=5632, heads=32, kv_heads=4, vocab=32000, layers=22, theta=10000.0)


def test_tinyllama_greedy_128_tokens(device):
    model, oracle = gpu_model_and_oracle(TINYLLAMA, 4, 256, seed=0)
    prompt = np.random.default_rng(0).integers(0, TINYLLAMA["vocab"], (1, 32))
    print("TinyLlama: 22 layers, prompt 32, 128 greedy tokens", flush=True)
    ex = ParallelExecutor(0, 1, None, model)
    out = run(ex.generate(torch.from_numpy(prompt).cuda(), max_new_tokens=128, temperature=0.0))
    new = out[0, 32:].cpu().numpy()
    assert new.shape == (128,)
    assert ex.last_decode_path == "trunk"           # head_dim 64, 8 q heads per kv head: one launch per token
    # logits of every step from the GPU's own decode path (the whole-trunk launch and
    # the lm_head), teacher-forced on the same tokens: the same kernels on the same
    # inputs, so the same bits as during generation
    _, lgs = _decode_logits(model, torch.from_numpy(prompt).cuda(), 128, forced=new[None, :])
    gl = [lg[0] for lg in lgs]
    print("  oracle teacher-forced run", flush=True)
    _, ol = oracle.generate_greedy(prompt, 128, forced=new[None, :])
    errs = [rel(g, o[0]) for g, o in zip(gl, ol)]
    print("  per-step logits max-abs-rel: " + " ".join(f"{e:.3f}" for e in errs), flush=True)
    agree, worst = 0, 0.0
    for t, (g, o) in enumerate(zip(gl, ol)):
        o = o[0].astype(np.float64)
        err = rel(g, o)
        worst = max(worst, err)
        assert err <= DEEP_LOGIT_TOL, f"step {t}: logits max-abs-rel {err:.3e}"
        tok = int(new[t])
        assert o[tok] >= o.max() - 0.02 * np.abs(o).max(), f"step {t}: token {tok} not near the oracle's argmax"
        agree += int(tok == int(np.argmax(o)))
        # the generated token is the argmax of the GPU's own logits at that step
        assert g[tok] == g.max()
    # Exact argmax agreement is asserted where it is decided: a step whose oracle top-2
    # gap exceeds the 2 % margin must pick the oracle's token (the margin check above
    # implies it; counted here).  Steps with a smaller gap are near-ties of the
    # random-init logits, where two correct paths that round at different points may
    # pick either token; they are reported, not counted against the run.
    decided = [t for t, o in enumerate(ol) if np.diff(np.sort(o[0].astype(np.float64))[-2:])[0]
               > 0.02 * np.abs(o[0]).max()]
    miss = [t for t in decided if int(new[t]) != int(np.argmax(ol[t][0]))]
    print(f"  worst logits max-abs-rel {worst:.2e}, argmax agreement {agree}/128; {len(decided)} steps decided "
          f"by more than the margin, {len(miss)} of them missed; {128 - len(decided)} near-ties", flush=True)
    assert not miss, f"steps {miss}: the oracle's clear argmax was not picked"


# ---------------------------------------------------------------- Llama-3-8B, 32 layers

LLAMA8B = dict(hidden=4096, inter=14336, heads=32, kv_heads=8, vocab=128256, layers=32)


@pytest.fixture(scope="module")
def llama8b():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from tests.test_gpu_decode_trunk import build
    return build(LLAMA8B, 4, 2048 + 64, seed=21)


def test_llama8b_trunk_vs_per_op_full(llama8b):
    from tests.test_gpu_decode_trunk import compare_paths
    print("Llama-3-8B 32 layers: trunk vs per-op, prompt 2048, 256 steps", flush=True)
    worst = compare_paths(llama8b, 2048, steps=256, capacity=2048 + 256 + 32, tol=PATH_TOL_32)
    print(f"  worst logits max-abs-rel {worst:.2e}", flush=True)


def _decode_logits(model, ids, steps, forced=None, fused_trunk=True, keep=None):
    """Prefill ids [B, S], then ``steps`` greedy decode steps; returns (tokens
    [B, steps], logits list of [B, V] fp32).  With ``forced`` [B, steps] the token
    fed at each step is forced (teacher forcing) instead of the argmax.  With
    ``keep`` (a count), only the last ``keep`` steps' logits are returned; with a
    set of step indices, those steps' logits in order (every step's are checked
    finite on the device either way)."""
    B, S = ids.shape
    cache = model.new_cache(B, S + steps + 32)
    logits, _ = run(model.forward(ids, past_key_values=cache, use_cache=True, last_only=True))
    tokens = torch.zeros((B, steps + 2), dtype=torch.int32, device="cuda")
    dec = DecodeGraph(model, cache, tokens, use_graph=False, fused_trunk=fused_trunk)
    _lib.argmax(logits.reshape(B, -1), ids=dec.bufs.ids.view(-1), tokens=tokens, step=cache.counters[1:])
    _lib.add_i32(cache.counters[1:], 1, n=1)
    if keep is None:
        want = set(range(steps))
    elif isinstance(keep, int):
        want = set(range(steps - keep, steps))
    else:
        want = set(keep)
    out = [f32(logits.reshape(B, -1))] if 0 in want else []
    finite = torch.isfinite(logits.float()).all()
    for s in range(steps - 1):
        if forced is not None:
            dec.bufs.ids.copy_(torch.as_tensor(forced[:, s], dtype=torch.int32, device="cuda").view(B, 1))
        dec.run(1)
        finite &= torch.isfinite(dec.logits.float()).all()
        if s + 1 in want:
            out.append(f32(dec.logits.reshape(B, -1)))
    torch.cuda.synchronize()
    assert bool(finite), "non-finite logits"
    if dec.bufs.plan is not None:
        assert dec.bufs.plan.status() == 0, "a trunk launch gave up"
    return tokens[:, :steps].cpu().numpy(), out


def test_llama8b_batch16_identical_rows(llama8b):
    m = llama8b
    gen = torch.Generator(device="cuda")
    gen.manual_seed(22)
    one = torch.randint(0, m.vocab_size, (1, 2048), generator=gen, device="cuda")
    print("Llama-3-8B 32 layers: batch 16 of one 2048-token prompt, 8 steps", flush=True)
    toks16, lg16 = _decode_logits(m, one.repeat(16, 1), 8)
    for b in range(1, 16):
        assert np.array_equal(toks16[b], toks16[0]), f"row {b} tokens differ"
        for t, lg in enumerate(lg16):
            assert np.array_equal(lg[b], lg[0]), f"row {b} logits differ at step {t}"
    # batch 1, per-op path, fed the batch's tokens: the same logits within tolerance
    toks1, lg1 = _decode_logits(m, one, 8, forced=toks16[:1], fused_trunk=False)
    assert toks1[0, 0] == toks16[0, 0]
    for t in range(8):
        assert rel(lg16[t][0], lg1[t][0]) <= PATH_TOL_32, f"step {t}"


def test_llama8b_batch16_256_steps(llama8b):
    """Batch 16 of 16 different 2048-token prompts for the workload's 256 decode
    steps: finite throughout; rows 0, 7 and 15 against batch-1 per-op decode of
    their prompts fed the batch's tokens, at the last 4 positions (2300-2303)."""
    m = llama8b
    gen = torch.Generator(device="cuda")
    gen.manual_seed(24)
    ids = torch.randint(0, m.vocab_size, (16, 2048), generator=gen, device="cuda")
    print("Llama-3-8B 32 layers: batch 16, prompt 2048, 256 steps", flush=True)
    toks, lg = _decode_logits(m, ids, 256, keep=4)
    for b in (0, 7, 15):
        print(f"  row {b} vs batch 1", flush=True)
        _, lg1 = _decode_logits(m, ids[b:b + 1], 256, forced=toks[b:b + 1], fused_trunk=False, keep=4)
        for t in range(4):
            e = rel(lg[t][b], lg1[t][0])
            assert e <= PATH_TOL_32, f"row {b}, step {252 + t}: max-abs-rel {e:.3e}"


def test_llama8b_prefill_last_position_vs_incremental(llama8b):
    m = llama8b
    gen = torch.Generator(device="cuda")
    gen.manual_seed(23)
    ids = torch.randint(0, m.vocab_size, (1, 2048), generator=gen, device="cuda")
    full, _ = run(m.forward(ids, last_only=True))
    cache = m.new_cache(1, 2048 + 32)
    run(m.forward(ids[:, :2047], past_key_values=cache, use_cache=True, last_only=True))
    step, _ = run(m.forward(ids[:, 2047:], past_key_values=cache, use_cache=True))
    err = rel(f32(step)[0], f32(full)[0])
    print(f"Llama-3-8B: prefill last position vs incremental, max-abs-rel {err:.2e}", flush=True)
    assert err <= PATH_TOL_32


# ---------------------------------------------------------------- Llama-3-70B rank-0 shard

def _shard_70b(bits, layers=80, seed=31, with_oracle_layer0=False):
    """The rank-0-of-8 shard of the Llama-3-70B shape; optionally layer 0's packed
    weights on the host in oracle form."""
    dev = torch.device("cuda", 0)
    H, heads, kv, I, V, ws = 8192, 64, 8, 28672, 128256, 8
    D = H // heads
    nq, nkv, Il, Vl = heads // ws * D, kv // ws * D, I // ws, V // ws
    m = ParallelTransformer(vocab_size=V, hidden_size=H, num_layers=layers, num_heads=heads, intermediate_size=I,
                            world_size=ws, rank=0, communicator=IdentityCommunicator(0, ws), num_kv_heads=kv,
                            max_position_embeddings=1024 + 64, rms_norm_eps=1e-5, rope_base=500000.0,
                            use_quantized=True, quantization_bits=bits, quantization_group_size=64,
                            embedding="vocab", quantized_lm_head=True, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def q(n, k):
        return _lib.quantize(torch.randn((n, k), generator=g, device=dev).mul_(0.02), bits=bits)

    def ql(t):
        return QLinear(host_u32(t[0]), host_u16(t[1]), host_u16(t[2]))

    layer0 = None
    for i, layer in enumerate(m.layers):
        li = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
        lp = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
        layer.input_layernorm.load_weights(li)
        layer.post_attention_layernorm.load_weights(lp)
        wq, wk, wv, wo = q(nq, H), q(nkv, H), q(nkv, H), q(H, nq)
        layer.attention.load_quantized_shards(*wq, None, *wk, None, *wv, None, *wo, None)
        wg, wu, wd = q(Il, H), q(Il, H), q(H, Il)
        layer.mlp.load_quantized_shards(*wu, None, *wd, None, *wg, None)
        if i == 0 and with_oracle_layer0:
            layer0 = dict(input_ln=host_u16(li), post_ln=host_u16(lp), q=ql(wq), k=ql(wk), v=ql(wv), o=ql(wo),
                          gate=ql(wg), up=ql(wu), down=ql(wd))
    m.load_embedding_weights(torch.randn((Vl, H), generator=g, device=dev).mul_(0.02).to(torch.bfloat16))
    m.load_norm_weights((1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16))
    m.load_quantized_lm_head_weights(*q(Vl, H))
    torch.cuda.synchronize()
    return m, layer0


@pytest.mark.parametrize("bits", [4, 8])
def test_llama70b_rank0_shard(device, bits):
    print(f"70B rank-0 shard W{bits}: 80 layers, batch 32, prefill 1024, 128 steps", flush=True)
    m, L0 = _shard_70b(bits, with_oracle_layer0=True)
    att = m.layers[0].attention
    assert (att.local_num_heads, att.local_num_kv_heads, m.layers[0].mlp.local_intermediate) == (8, 1, 3584)
    # layer 0 (a rank's partial: o_proj and down_proj outputs before the all-reduce)
    # against the oracle on the same packed weights
    sh = DecoderShape(vocab_size=16, hidden_size=8192, num_layers=1, num_heads=8, num_kv_heads=1,
                      intermediate_size=3584, head_dim=128, rope_theta=500000.0, bits=bits)
    rng = np.random.default_rng(32)
    x = rng.standard_normal((2, 12, 8192)).astype(np.float32)
    from oracle.bf16 import f32_to_bf16, round_bf16
    xb = f32_to_bf16(x)
    h, _ = run(m.layers[0].forward(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()))
    o = OracleDecoder(sh, dict(layers=[L0]))
    x32 = bf16_to_f32(xb)
    xn = rms_norm(x32, L0["input_ln"], sh.rms_norm_eps)
    hr = round_bf16(x32 + o._attn(0, xn, L0))
    xn = rms_norm(hr, L0["post_ln"], sh.rms_norm_eps)
    hr = round_bf16(hr + o._mlp(xn, L0))
    err = rel(bf16_to_f32(host_u16(h)).reshape(hr.shape), hr)
    print(f"  layer 0 vs oracle: max-abs-rel {err:.2e}", flush=True)
    assert err <= LOGIT_TOL
    # batch-32 decode after a 1024-token prefill; row 5 against batch 1 of its prompt
    gen = torch.Generator(device="cuda")
    gen.manual_seed(33)
    ids = torch.randint(0, 128256, (32, 1024), generator=gen, device="cuda")
    at = [0, 1, 2, 4, 8, 16, 32, 48, 64, 80, 96, 112, 120, 124, 126, 127]
    toks, lg = _decode_logits(m, ids, 128, keep=at)
    toks1, lg1 = _decode_logits(m, ids[5:6], 128, forced=toks[5:6], keep=at)
    errs = [rel(a[5], b[0]) for a, b in zip(lg, lg1)]
    rms = [float(np.sqrt(np.mean((a[5].astype(np.float64) - b[0]) ** 2) / np.mean(b[0].astype(np.float64) ** 2)))
           for a, b in zip(lg, lg1)]
    print("  batch 32 row 5 vs batch 1, by step: " + " ".join(f"{t}:{e:.3f}/{r:.4f}" for t, e, r in zip(at, errs, rms)),
          flush=True)
    for t, e, r in zip(at, errs, rms):
        assert e <= PATH_TOL_80, f"step {t}: batch-32 row 5 vs batch 1, max-abs-rel {e:.3e}"
        assert r <= PATH_RMS_80, f"step {t}: batch-32 row 5 vs batch 1, rms-relative {r:.3e}"
    # rounding drift between two correct paths does not grow along the cache; a slot or
    # length error past some position would
    assert np.mean(rms[-4:]) <= 1.5 * np.mean(rms[1:5]), "difference grows with the position"
