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
