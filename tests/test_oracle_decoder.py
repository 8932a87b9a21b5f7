"""Pins oracle/decoder.py (the numpy restatement of the layer wiring)."""
import numpy as np

from oracle.bf16 import bf16_to_f32, f32_to_bf16, round_bf16
from oracle.decoder import (DecoderShape, OracleDecoder, apply_rope, attention_core,
                            random_decoder_weights, rms_norm, rope_cos_sin)


def test_rms_norm_closed_form():
    c = np.array([[0.5] * 8, [-3.0] * 8], np.float32)
    w = f32_to_bf16(np.linspace(0.5, 2.0, 8).astype(np.float32))
    y = rms_norm(c, w, 1e-5)
    expect = np.sign(c) * np.abs(c) / np.sqrt(c * c + 1e-5) * bf16_to_f32(w)
    assert np.allclose(y, round_bf16(expect.astype(np.float32)), rtol=0, atol=0)


def test_rope_equals_complex_rotation():
    rng = np.random.default_rng(0)
    D, S, base = 16, 7, 10000.0
    x = round_bf16(rng.standard_normal((1, 2, S, D)).astype(np.float32))
    pos = np.arange(5, 5 + S)
    cos, sin = rope_cos_sin(pos, D, base)
    got = apply_rope(x, cos, sin)
    # pair (x_i, x_{i+D/2}) rotates as the complex number x_i + i x_{i+D/2} by angle t*theta_i
    theta = base ** (-np.arange(0, D, 2) / D)
    z = (x[..., : D // 2] + 1j * x[..., D // 2:]) * np.exp(1j * np.outer(pos, theta))[None, None]
    ref = np.concatenate([z.real, z.imag], -1)
    assert np.allclose(got, ref, atol=2e-2, rtol=1e-2)
    # rotation preserves the pair norms (up to bf16 rounding)
    n0 = np.hypot(x[..., : D // 2], x[..., D // 2:])
    n1 = np.hypot(got[..., : D // 2], got[..., D // 2:])
    assert np.allclose(n0, n1, rtol=2e-2, atol=1e-2)


def test_rope_position_zero_is_identity():
    rng = np.random.default_rng(1)
    x = round_bf16(rng.standard_normal((1, 1, 1, 8)).astype(np.float32))
    cos, sin = rope_cos_sin([0], 8, 10000.0)
    assert np.array_equal(apply_rope(x, cos, sin), x)


def test_attention_core_matches_loop():
    rng = np.random.default_rng(2)
    B, H, S, T, D = 1, 2, 3, 5, 4
    q = rng.standard_normal((B, H, S, D)).astype(np.float32)
    k = rng.standard_normal((B, H, T, D)).astype(np.float32)
    v = rng.standard_normal((B, H, T, D)).astype(np.float32)
    got = attention_core(q, k, v, 0.5, T - S)
    ref = np.zeros((B, H, S, D))
    for h in range(H):
        for i in range(S):
            allowed = [j for j in range(T) if j <= i + T - S]
            sc = np.array([0.5 * q[0, h, i] @ k[0, h, j] for j in allowed])
            p = np.exp(sc - sc.max())
            p /= p.sum()
            ref[0, h, i] = sum(p[n] * v[0, h, j] for n, j in enumerate(allowed))
    assert np.allclose(got, ref, atol=1e-2, rtol=1e-2)
    # single query (decode) attends to every cached key
    one = attention_core(q[:, :, -1:], k, v, 0.5, 0)
    assert np.allclose(one, got[:, :, -1:], atol=1e-6)


def _tiny_shape(layers=2):
    return DecoderShape(vocab_size=320, hidden_size=128, num_layers=layers, num_heads=4,
                        num_kv_heads=2, intermediate_size=192, rope_theta=10000.0)


def test_kv_cache_matches_full_sequence():
    sh = _tiny_shape()
    w = random_decoder_weights(sh, seed=0, std=0.05)
    ids = np.random.default_rng(3).integers(0, sh.vocab_size, size=(2, 9))
    full = OracleDecoder(sh, w).forward(ids)
    dec = OracleDecoder(sh, w)
    steps = [dec.forward(ids[:, :6])[:, -1]]
    for t in range(6, 9):
        steps.append(dec.forward(ids[:, t:t + 1])[:, -1])
    for n, t in enumerate(range(5, 9)):
        assert np.allclose(steps[n], full[:, t], atol=3e-2, rtol=3e-2)


def test_gqa_equals_explicit_head_sharing():
    sh = _tiny_shape(1)
    w = random_decoder_weights(sh, seed=1, std=0.05)
    ids = np.random.default_rng(4).integers(0, sh.vocab_size, size=(1, 5))
    # expand K/V projections to one KV head per query head (MHA) by duplicating rows
    import copy
    w2 = copy.deepcopy(w)
    D = sh.head_dim
    rep = sh.num_heads // sh.num_kv_heads
    for key in ("k", "v"):
        lin = w2["layers"][0][key]
        for name in ("wq", "scales", "biases"):
            arr = getattr(lin, name).reshape(sh.num_kv_heads, D, -1)
            setattr(lin, name, np.repeat(arr, rep, axis=0).reshape(sh.num_heads * D, -1))
        lin._w32 = None
    sh2 = DecoderShape(**{**sh.__dict__, "num_kv_heads": sh.num_heads})
    a = OracleDecoder(sh, w).forward(ids)
    b = OracleDecoder(sh2, w2).forward(ids)
    assert np.array_equal(a, b)


def test_teacher_forcing_with_own_tokens_reproduces_free_run():
    sh = _tiny_shape()
    w = random_decoder_weights(sh, seed=2, std=0.05)
    ids = np.random.default_rng(5).integers(0, sh.vocab_size, size=(1, 4))
    toks, logits = OracleDecoder(sh, w).generate_greedy(ids, 5)
    toks2, logits2 = OracleDecoder(sh, w).generate_greedy(ids, 5, forced=toks[:, 4:])
    assert np.array_equal(toks, toks2)
    for a, b in zip(logits, logits2):
        assert np.array_equal(a, b)


# ---------------------------------------------------------------- wiring pins
#
# Closed forms on structured weights.  Each expectation is computed in float64
# from the formula the reference states (pre-norm block transformer.py:237-254,
# SwiGLU mlp.py:161-162 and :241-254, model transformer.py:536-577, attention
# attention.py:403-471), without calling oracle.decoder; alternatives a
# plausible wiring mistake would compute are shown to miss by far more than the
# tolerance.

from oracle.decoder import QLinear, silu  # noqa: E402
from oracle.mlx_affine import pack  # noqa: E402


def _structured(q_codes, scale, bits=4, group_size=64):
    """QLinear with W = scale * q (bias 0): integer codes [N, K], one scale for all groups."""
    N, K = q_codes.shape
    s = np.full((N, K // group_size), f32_to_bf16(np.float32(scale)), np.uint16)
    b = np.zeros_like(s)
    return QLinear(pack(q_codes, bits), s, b)


def _eye(n, k, code=1, scale=1.0):
    q = np.zeros((n, k), np.uint32)
    m = min(n, k)
    q[np.arange(m), np.arange(m)] = code
    return _structured(q, scale)


def _zero(n, k):
    return _structured(np.zeros((n, k), np.uint32), 0.0)


def _norm64(x, w, eps=1e-5):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _silu64(x):
    return x / (1.0 + np.exp(-np.asarray(x, np.float64)))


def _close(got, exp, frac=2e-2):
    return float(np.abs(got - exp).max()) <= frac * float(np.abs(exp).max())


def test_silu_known_values():
    x = np.array([0.0, 1.0, -1.0, 2.5, 30.0, -30.0, 100.0, -100.0], np.float32)
    got = silu(x)
    exp = np.array([0.0, 1 / (1 + np.exp(-1.0)), -1 / (1 + np.exp(1.0)), 2.5 / (1 + np.exp(-2.5)),
                    30.0, -30.0 * np.exp(-30.0), 100.0, -100.0 * np.exp(-100.0)])
    assert got[0] == 0.0
    assert np.allclose(got, exp, rtol=1e-6, atol=1e-30)
    assert abs(got[1] - 0.7310585786300049) < 1e-6
    assert got[7] <= 0.0 and np.isfinite(got[7])


H64 = 64


def _one_layer_weights(rng, o_zero=True, down=None):
    """hidden = intermediate = 64, 2 q heads / 1 kv head of 32, vocab 96."""
    sh = DecoderShape(vocab_size=96, hidden_size=H64, num_layers=1, num_heads=2, num_kv_heads=1,
                      intermediate_size=H64, rope_theta=10000.0)
    nw = lambda: f32_to_bf16((1.0 + 0.2 * rng.standard_normal(H64)).astype(np.float32))  # noqa: E731
    rq = lambda n, k: QLinear(*__import__("oracle.mlx_affine", fromlist=["x"]).quantize_bf16(  # noqa: E731
        (0.05 * rng.standard_normal((n, k))).astype(np.float32), 64, 4))
    L = dict(input_ln=nw(), post_ln=nw(), q=rq(64, 64), k=rq(32, 64), v=rq(32, 64),
             o=_zero(64, 64) if o_zero else rq(64, 64),
             gate=_eye(64, 64, code=2), up=_eye(64, 64, code=1),
             down=_eye(64, 64, code=1) if down is None else down)
    # rms 4 rows: far from their normalisation, so norm(h) and h differ
    embed = f32_to_bf16((4.0 * rng.standard_normal((96, H64))).astype(np.float32))
    W = dict(embed=embed, norm=nw(), lm_head=_eye(96, 64, code=1), layers=[L])
    return sh, W


def test_block_is_identity_when_o_and_down_are_zero():
    rng = np.random.default_rng(30)
    sh, W = _one_layer_weights(rng, o_zero=True, down=_zero(64, 64))
    dec = OracleDecoder(sh, W)
    h = round_bf16(rng.standard_normal((1, 5, H64)).astype(np.float32))
    L = W["layers"][0]
    from oracle.decoder import rms_norm as _rms
    xn = _rms(h, L["input_ln"], sh.rms_norm_eps)
    h1 = round_bf16(h + dec._attn(0, xn, L))
    xn = _rms(h1, L["post_ln"], sh.rms_norm_eps)
    h2 = round_bf16(h1 + dec._mlp(xn, L))
    assert np.array_equal(h1, h) and np.array_equal(h2, h)
    # the whole model: logits = norm(embedding row) through the identity lm_head
    ids = np.array([[3, 17, 95]])
    logits = OracleDecoder(sh, W).forward(ids)
    exp = _norm64(bf16_to_f32(W["embed"][ids]), bf16_to_f32(W["norm"]))
    exp = np.concatenate([exp, np.zeros(exp.shape[:-1] + (32,))], -1)   # vocab rows 64..95 are zero
    assert _close(logits, exp, 1e-2)


def test_mlp_gate_up_roles():
    rng = np.random.default_rng(31)
    sh, W = _one_layer_weights(rng)
    # inputs in [-4, 1.5]: for large positive x every variant tends to 2 x^2, so
    # the roles show where the sigmoid is far from 1
    x = round_bf16(np.stack([np.linspace(-4, 1.5, H64), np.linspace(1.5, -4, H64),
                             rng.uniform(-4, 1.5, H64)]).astype(np.float32))
    got = OracleDecoder(sh, W)._mlp(x, W["layers"][0])
    xd = x.astype(np.float64)
    exp = _silu64(2 * xd) * xd                       # gate = 2I, up = I, down = I
    swapped = _silu64(xd) * 2 * xd                   # gate and up exchanged
    ungated = _silu64(2 * xd)                        # up dropped
    assert _close(got, exp, 1e-2)
    assert not _close(swapped, exp, 0.1) and not _close(ungated, exp, 0.1)


def test_one_layer_model_closed_form_prenorm():
    rng = np.random.default_rng(32)
    sh, W = _one_layer_weights(rng)                  # o = 0: the attention adds nothing
    ids = np.array([[5, 60, 7, 33]])
    logits = OracleDecoder(sh, W).forward(ids)[..., :H64]
    L = W["layers"][0]
    w_post, w_fin = bf16_to_f32(L["post_ln"]).astype(np.float64), bf16_to_f32(W["norm"]).astype(np.float64)
    h = bf16_to_f32(W["embed"][ids]).astype(np.float64)
    xn = _norm64(h, w_post)
    exp = _norm64(h + _silu64(2 * xn) * xn, w_fin)                 # pre-norm block, final norm, lm_head = I
    w_in = bf16_to_f32(L["input_ln"]).astype(np.float64)
    h1 = _norm64(h, w_in)                                           # post-norm: norm after each residual add
    post_norm = _norm64(_norm64(h1 + _silu64(2 * h1) * h1, w_post), w_fin)
    no_resid = _norm64(_silu64(2 * xn) * xn, w_fin)                 # residual dropped
    no_final = h + _silu64(2 * xn) * xn                             # final norm missing
    no_mlp = _norm64(h, w_fin)                                      # block output dropped
    assert _close(logits, exp, 2e-2)
    for wrong in (post_norm, no_resid, no_final, no_mlp):
        assert not _close(wrong, exp, 0.1)


def test_attention_value_path_and_gqa_mapping():
    # v = I on the kv head's slice, o = I: at one token the softmax is over one
    # key, so query head h outputs v of kv head h // rep = x[(h // rep) * D : ...]
    rng = np.random.default_rng(33)
    sh = DecoderShape(vocab_size=64, hidden_size=128, num_layers=1, num_heads=4, num_kv_heads=2,
                      intermediate_size=64, rope_theta=10000.0)
    D = sh.head_dim                                   # 32
    rq = lambda n, k: QLinear(*__import__("oracle.mlx_affine", fromlist=["x"]).quantize_bf16(  # noqa: E731
        (0.05 * rng.standard_normal((n, k))).astype(np.float32), 64, 4))
    L = dict(q=rq(128, 128), k=rq(64, 128), v=_eye(64, 128), o=_eye(128, 128))
    dec = OracleDecoder(sh, dict(layers=[L]))
    x = round_bf16(rng.standard_normal((1, 1, 128)).astype(np.float32))
    got = dec._attn(0, x, L)[0, 0]
    exp = np.concatenate([x[0, 0, (h // 2) * D:(h // 2 + 1) * D] for h in range(4)])
    wrong = np.concatenate([x[0, 0, (h % 2) * D:(h % 2 + 1) * D] for h in range(4)])   # heads interleaved
    assert np.array_equal(got, exp)
    assert not np.array_equal(wrong, exp)


def test_attention_causal_uniform_scores():
    # q = 0: every allowed score is 0, so position i outputs the mean of v over
    # positions 0..i (causal); a mask of the wrong orientation would average the
    # future, no mask would give the full mean everywhere
    rng = np.random.default_rng(34)
    sh = DecoderShape(vocab_size=64, hidden_size=64, num_layers=1, num_heads=2, num_kv_heads=1,
                      intermediate_size=64, rope_theta=10000.0)
    rq = lambda n, k: QLinear(*__import__("oracle.mlx_affine", fromlist=["x"]).quantize_bf16(  # noqa: E731
        (0.05 * rng.standard_normal((n, k))).astype(np.float32), 64, 4))
    L = dict(q=_zero(64, 64), k=rq(32, 64), v=_eye(32, 64), o=_eye(64, 64))
    x = round_bf16(rng.standard_normal((1, 6, 64)).astype(np.float32))
    got = OracleDecoder(sh, dict(layers=[L]))._attn(0, x, L)[0]
    v = x[0, :, :32].astype(np.float64)
    run_mean = np.cumsum(v, 0) / np.arange(1, 7)[:, None]
    exp = np.concatenate([run_mean, run_mean], -1)     # both q heads share kv head 0
    assert _close(got, exp, 1e-2)
    fut = np.cumsum(v[::-1], 0)[::-1] / np.arange(6, 0, -1)[:, None]
    assert not _close(np.concatenate([fut, fut], -1), exp, 0.1)
    full = np.repeat(v.mean(0, keepdims=True), 6, 0)
    assert not _close(np.concatenate([full, full], -1), exp, 0.1)
    # and the cache: the same positions fed one at a time give the same outputs
    dec = OracleDecoder(sh, dict(layers=[L]))
    inc = np.concatenate([dec._attn(0, x[:, t:t + 1], L)[0] for t in range(6)])
    assert _close(inc, exp, 1e-2)


def _mask_case(seed, T=9, D=8):
    rng = np.random.default_rng(seed)
    q = round_bf16(rng.standard_normal((1, 2, 1, D)).astype(np.float32))
    k = round_bf16(rng.standard_normal((1, 2, T, D)).astype(np.float32))
    v = round_bf16(rng.standard_normal((1, 2, T, D)).astype(np.float32))
    return q, k, v


def test_attention_mask_zero_and_row_constant_are_no_ops():
    # softmax is invariant to a per-row shift: a mask constant along the keys changes
    # nothing (a mask applied after the softmax, or multiplied in, would)
    q, k, v = _mask_case(2)
    base = attention_core(q, k, v, 0.35, k.shape[2] - 1)
    assert np.array_equal(attention_core(q, k, v, 0.35, k.shape[2] - 1, mask=np.zeros((1, 1, 1, 9))), base)
    shifted = attention_core(q, k, v, 0.35, k.shape[2] - 1, mask=np.full((1, 2, 1, 1), -3.0))
    assert np.allclose(shifted, base, atol=1e-6, rtol=0)


def test_attention_mask_minus_inf_drops_the_key():
    # -inf at key j for one position equals attending without key j
    q, k, v = _mask_case(3)
    j = 4
    m = np.zeros((1, 1, 1, 9), np.float32)
    m[..., j] = -np.inf
    got = attention_core(q, k, v, 0.35, 8, mask=m)
    keep = [i for i in range(9) if i != j]
    ref = attention_core(q, k[:, :, keep], v[:, :, keep], 0.35, 7)
    assert np.allclose(got, ref, atol=1e-6, rtol=0)


def test_attention_mask_log2_doubles_a_key():
    # adding log 2 to key j's scaled score equals key j appearing twice (a mask scaled
    # with the scores, or subtracted, would not)
    q, k, v = _mask_case(4)
    j = 2
    m = np.zeros((1, 1, 1, 9), np.float32)
    m[..., j] = np.log(2.0)
    got = attention_core(q, k, v, 0.35, 8, mask=m)
    dup = [0, 1, 2, 2, 3, 4, 5, 6, 7, 8]
    ref = attention_core(q, k[:, :, dup], v[:, :, dup], 0.35, 9)
    assert np.allclose(got, ref, atol=1e-6, rtol=0)


# ---------------------------------------------------------------- the other MLP and norm forms

def test_activation_closed_forms_and_library():
    import math
    from oracle.decoder import activation
    x = np.linspace(-6, 6, 2001).astype(np.float32)
    x64 = x.astype(np.float64)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x64])    # Python's math.erf
    ge = activation(x, "gelu_exact")
    assert np.abs(ge - exact).max() <= 2e-6 * max(1.0, np.abs(exact).max())
    # the tanh form is within 5e-4 of the exact GELU (its published accuracy), the
    # sigmoid form within 0.021; a wrong constant misses either bound
    assert np.abs(activation(x, "gelu_new") - exact).max() <= 5e-4
    assert np.abs(activation(x, "gelu") - exact).max() <= 0.021
    assert np.abs(activation(x, "gelu") - x64 / (1 + np.exp(-1.702 * x64))).max() <= 1e-6 * 6
    t = np.tanh(0.7978845608028654 * (x64 + 0.044715 * x64 ** 3))
    assert np.abs(activation(x, "gelu_new") - 0.5 * x64 * (1 + t)).max() <= 2e-6 * 6
    for name in ("gelu", "gelu_new", "gelu_exact", "silu", "swish"):
        y = activation(np.array([0.0, 30.0, -30.0], np.float32), name)
        assert y[0] == 0.0 and abs(y[1] - 30.0) < 1e-4 and abs(y[2]) < 1e-3
    r = activation(np.array([-2.0, -0.0, 0.0, 3.0, np.nan], np.float32), "relu")
    assert r[0] == 0.0 and r[1] == 0.0 and r[2] == 0.0 and r[3] == 3.0 and np.isnan(r[4])
    assert np.array_equal(activation(x, "swish"), activation(x, "silu"))
    import pytest
    with pytest.raises(ValueError):
        activation(x, "tanh")


def test_rms_norm_bias_is_added_after_rounding():
    rng = np.random.default_rng(40)
    x = round_bf16(rng.standard_normal((3, 64)).astype(np.float32) * 3)
    w = f32_to_bf16((1 + 0.1 * rng.standard_normal(64)).astype(np.float32))
    b = f32_to_bf16((0.5 * rng.standard_normal(64)).astype(np.float32))
    y0 = rms_norm(x, w, 1e-5)
    assert np.array_equal(rms_norm(x, w, 1e-5, b), round_bf16(y0 + bf16_to_f32(b)))
    # constant rows: the normalised row is w (closed form), plus the bias
    c = np.full((2, 64), 2.5, np.float32)
    exp = bf16_to_f32(w).astype(np.float64) * 2.5 / np.sqrt(2.5 ** 2 + 1e-5) + bf16_to_f32(b)
    assert np.abs(rms_norm(c, w, 1e-5, b) - exp).max() <= 2 ** -7 * np.abs(exp).max()


def test_ungated_and_other_activation_mlp_roles():
    from oracle.decoder import activation
    rng = np.random.default_rng(41)
    sh, W = _one_layer_weights(rng)                  # gate = 2I, up = I, down = I
    L = W["layers"][0]
    x = round_bf16(np.stack([np.linspace(-4, 2, H64), rng.uniform(-4, 2, H64)]).astype(np.float32))
    xd = x.astype(np.float64)
    for name in ("gelu", "gelu_new", "relu", "gelu_exact"):
        sh.activation, sh.gated = name, True
        got = OracleDecoder(sh, W)._mlp(x, L)
        f2 = activation((2 * x).astype(np.float32), name).astype(np.float64)
        assert _close(got, f2 * xd, 1e-2), name                          # f(gate) * up
        sh.gated = False
        got = OracleDecoder(sh, W)._mlp(x, L)
        f1 = activation(x, name).astype(np.float64)
        assert _close(got, f1, 1e-2), name                               # f(up), the gate ignored
        assert not _close(got, f2 * xd, 0.1), name
