"""The MLP and norm forms beside the Llama family's gated SiLU and plain RMSNorm
(``parallel/mlp.py:159-180, 236-250``; ``transformer.py:57-59``), on the GPU against
the oracle:

* ``sc_act_bf16``: every activation, gated and ungated, within one bf16 step of the
  oracle on < 1 % of elements (the device's exp / tanh / erf and numpy's may differ
  in the last fp32 bit, which moves a rare rounding), and NaN / 0 / large inputs;
  the gated SiLU bit-identical to ``sc_silu_mul_bf16``;
* ``sc_add_row_bias_bf16``: bit-exact (one bf16 addition);
* ``ParallelMLP`` gated and ungated with each activation against the oracle's MLP on
  the same packed weights (1e-2);
* ``RMSNorm`` with a bias, and a two-layer model with norm biases and the ungated
  ``gelu_new`` MLP (the Phi-2 names the loader maps, in the reference's sequential
  block): logits against the oracle decoder, and greedy decode through the executor
  (the per-op path: the whole-trunk launch takes only the bias-free gated SiLU).
"""
import asyncio

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16, round_bf16
from oracle.decoder import DecoderShape, OracleDecoder, QLinear, activation, rms_norm
from shardcompute_amd import _lib
from shardcompute_amd.decode_plan import eligible
from shardcompute_amd.executor import ParallelExecutor
from shardcompute_amd.parallel.mlp import ParallelMLP
from shardcompute_amd.parallel.transformer import ParallelTransformer, RMSNorm
from tests.gpu_util import LINEAR_TOL, bf16_ulp_diff, dev_bf16, host_u16, host_u32, max_abs_rel

pytestmark = pytest.mark.gpu

KINDS = ("silu", "gelu", "gelu_new", "relu", "gelu_exact")


def _inputs(rng, rows, I):
    x = (rng.standard_normal((rows, I)) * 3).astype(np.float32)
    x[0, :8] = [0.0, -0.0, 40.0, -40.0, 1e-3, -1e-3, 8.5, -8.5]
    return f32_to_bf16(x)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("gated", [True, False])
def test_act_matches_oracle(device, kind, gated):
    rng = np.random.default_rng(KINDS.index(kind) + 10 * gated)
    rows, I = 37, 1032
    x = _inputs(rng, rows, 2 * I if gated else I)
    print(f"act {kind} gated={gated}", flush=True)
    y = host_u16(_lib.act(dev_bf16(x), kind, gated=gated))
    torch.cuda.synchronize()
    xf = bf16_to_f32(x)
    ref = activation(xf[:, :I], kind) * (xf[:, I:] if gated else np.float32(1))
    r = f32_to_bf16(ref.astype(np.float32))
    # where 1 + tanh or 1 + erf cancels (large negative x) both sides hold fp32 noise
    # far below the output's scale: those elements are compared absolutely
    rf, yf = bf16_to_f32(r).astype(np.float64), bf16_to_f32(y).astype(np.float64)
    scale = np.abs(rf).max()
    d = bf16_ulp_diff(y, r)
    bad = (d > 1) & (np.abs(yf - rf) > 1e-5 * scale)
    assert not bad.any(), (kind, gated, int(bad.sum()))
    sig = np.abs(rf) >= 1e-4 * scale
    assert d[sig].max() <= 1 and (d[sig] > 0).mean() < 0.01, (kind, gated, d[sig].max(), (d[sig] > 0).mean())


def test_act_nan_and_in_place(device):
    x = f32_to_bf16(np.array([[np.nan, 1.0, -2.0, 0.0, 3.0, -0.5, 7.0, np.inf]], np.float32))
    for kind in KINDS:
        y = host_u16(_lib.act(dev_bf16(x), kind, gated=False))
        assert np.isnan(bf16_to_f32(y)[0, 0]), kind
    t = dev_bf16(x)
    _lib.act(t, "relu", gated=False, out=t)           # ungated in place
    torch.cuda.synchronize()
    assert bf16_to_f32(host_u16(t))[0, 2] == 0.0 and bf16_to_f32(host_u16(t))[0, 4] == 3.0


def test_gated_silu_equals_silu_mul(device):
    rng = np.random.default_rng(3)
    gu = dev_bf16(_inputs(rng, 19, 2 * 1536))
    a = _lib.act(gu, "silu", gated=True)
    b = _lib.silu_mul(gu)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_add_row_bias_bit_exact(device):
    rng = np.random.default_rng(4)
    x = _inputs(rng, 5, 2048)
    b = f32_to_bf16(rng.standard_normal(2048).astype(np.float32))
    y = host_u16(_lib.add_row_bias(dev_bf16(x), dev_bf16(b)))
    torch.cuda.synchronize()
    assert np.array_equal(y, f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(b)[None]))


def _q(g, n, k, bits=4):
    t = _lib.quantize(torch.randn((n, k), generator=g, device="cuda").mul_(0.02), bits=bits)
    return t, QLinear(host_u32(t[0]), host_u16(t[1]), host_u16(t[2]))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("gated", [True, False])
def test_mlp_forms_match_oracle(device, kind, gated):
    H, I, rows = 1024, 2816, 6
    g = torch.Generator(device="cuda")
    g.manual_seed(50 + KINDS.index(kind))
    mlp = ParallelMLP(H, I, 1, 0, activation=kind, use_gated=gated, use_quantized=True)
    (ut, uo), (dt, do) = _q(g, I, H), _q(g, H, I)
    gate = _q(g, I, H) if gated else None
    mlp.load_quantized_shards(*ut, None, *dt, None, *(gate[0] if gated else (None, None, None)), None)
    x = torch.randn((rows, H), generator=g, device="cuda").mul_(2).to(torch.bfloat16)
    print(f"MLP {kind} gated={gated}", flush=True)
    y = asyncio.run(mlp.forward(x))
    torch.cuda.synchronize()
    sh = DecoderShape(vocab_size=8, hidden_size=H, num_layers=1, num_heads=8, num_kv_heads=8, intermediate_size=I,
                      activation=kind, gated=gated)
    L = dict(up=uo, down=do, gate=gate[1] if gated else None)
    ref = OracleDecoder(sh, dict(layers=[L]))._mlp(bf16_to_f32(host_u16(x)), L)
    assert max_abs_rel(host_u16(y), ref) <= LINEAR_TOL


def test_rms_norm_with_bias(device):
    rng = np.random.default_rng(5)
    x = _inputs(rng, 7, 2048)
    r = _inputs(rng, 7, 2048)
    w = f32_to_bf16((1 + 0.1 * rng.standard_normal(2048)).astype(np.float32))
    b = f32_to_bf16((0.3 * rng.standard_normal(2048)).astype(np.float32))
    n = RMSNorm(2048, eps=1e-5)
    n.load_weights(dev_bf16(w), dev_bf16(b))
    assert not n.fusable
    h = torch.empty((7, 2048), dtype=torch.bfloat16, device="cuda")
    y = host_u16(n(dev_bf16(x), residual=dev_bf16(r), h_out=h))
    torch.cuda.synchronize()
    hr = f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(r))
    assert np.array_equal(host_u16(h), hr)
    ref = f32_to_bf16(rms_norm(bf16_to_f32(hr), w, 1e-5, b))
    d = bf16_ulp_diff(y, ref)
    assert d.max() <= 1 and (d > 0).mean() < 0.01


def _phi_style_model(bits=4, layers=2, seed=60):
    """hidden 1024, 16 heads of 64, intermediate 4096, ungated gelu_new MLP, norms with
    biases, vocab 2048; the same weights in oracle form."""
    H, I, V, heads = 1024, 4096, 2048, 16
    dev = torch.device("cuda", 0)
    m = ParallelTransformer(vocab_size=V, hidden_size=H, num_layers=layers, num_heads=heads, intermediate_size=I,
                            world_size=1, rank=0, max_position_embeddings=256, rms_norm_eps=1e-5,
                            rope_base=10000.0, mlp_activation="gelu_new", use_gated_mlp=False, use_quantized=True,
                            quantization_bits=bits, embedding="vocab", quantized_lm_head=True, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def nw(scale):
        t = (scale * torch.randn(H, generator=g, device=dev) + (1.0 if scale < 0.5 else 0.0)).to(torch.bfloat16)
        return t, host_u16(t)

    Ls = []
    for layer in m.layers:
        (li, li_h), (lib_, lib_h) = nw(0.1), nw(0.5)
        (lp, lp_h), (lpb, lpb_h) = nw(0.1), nw(0.5)
        layer.input_layernorm.load_weights(li, lib_)
        layer.post_attention_layernorm.load_weights(lp, lpb)
        (qt, qo), (kt, ko), (vt, vo), (ot, oo) = _q(g, H, H, bits), _q(g, H, H, bits), _q(g, H, H, bits), \
            _q(g, H, H, bits)
        layer.attention.load_quantized_shards(*qt, None, *kt, None, *vt, None, *ot, None)
        (ut, uo), (dt, do) = _q(g, I, H, bits), _q(g, H, I, bits)
        layer.mlp.load_quantized_shards(*ut, None, *dt, None)
        Ls.append(dict(input_ln=li_h, input_ln_bias=lib_h, post_ln=lp_h, post_ln_bias=lpb_h, q=qo, k=ko, v=vo,
                       o=oo, up=uo, down=do))
    emb = torch.randn((V, H), generator=g, device=dev).mul_(0.02).to(torch.bfloat16)
    m.load_embedding_weights(emb)
    (fn, fn_h), (fb, fb_h) = nw(0.1), nw(0.5)
    m.norm.load_weights(fn, fb)
    lm_t, lm_o = _q(g, V, H, bits)
    m.load_quantized_lm_head_weights(*lm_t)
    torch.cuda.synchronize()
    sh = DecoderShape(vocab_size=V, hidden_size=H, num_layers=layers, num_heads=heads, num_kv_heads=heads,
                      intermediate_size=I, rope_theta=10000.0, bits=bits, activation="gelu_new", gated=False)
    W = dict(embed=host_u16(emb), norm=fn_h, norm_bias=fb_h, lm_head=lm_o, layers=Ls)
    return m, OracleDecoder(sh, W)


def test_norm_bias_ungated_gelu_new_model_matches_oracle(device):
    m, o = _phi_style_model()
    ids = np.random.default_rng(61).integers(0, 2048, (2, 23))
    print("norm-bias / ungated gelu_new model: prefill of 2 x 23 against the oracle", flush=True)
    logits, _ = asyncio.run(m.forward(torch.from_numpy(ids).cuda()))
    torch.cuda.synchronize()
    ref = o.forward(ids)
    assert max_abs_rel(host_u16(logits.reshape(-1, 2048)), ref.reshape(-1, 2048)) <= 3e-2
    # greedy decode through the executor: the per-op path, tokens within the oracle's margin
    assert eligible(m, m.new_cache(1, 64))[0] is False
    ex = ParallelExecutor(0, 1, None, m)
    prompt = ids[:1, :10]
    out = asyncio.run(ex.generate(torch.from_numpy(prompt).cuda(), max_new_tokens=12, temperature=0.0))
    assert ex.last_decode_path == "per-op"
    new = out[0, 10:].cpu().numpy()
    _, ol = o.generate_greedy(prompt, 12, forced=new[None, :])
    for t, lo in enumerate(ol):
        lo = lo[0].astype(np.float64)
        assert lo[int(new[t])] >= lo.max() - 0.02 * np.abs(lo).max(), f"step {t}"
