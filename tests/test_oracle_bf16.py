"""Pins oracle/bf16.py: exhaustive round trip and agreement with torch's RNE cast."""
import numpy as np
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16


def test_exhaustive_round_trip():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    back = f32_to_bf16(bf16_to_f32(h))
    f = bf16_to_f32(h)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], h[~nan])
    # NaNs stay NaN and keep their sign
    assert np.all(np.isnan(bf16_to_f32(back[nan])))
    assert np.array_equal(back[nan] & 0x8000, h[nan] & 0x8000)


def _torch_bf16_bits(f):
    t = torch.from_numpy(np.ascontiguousarray(f, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_matches_torch_rne_random():
    rng = np.random.default_rng(0)
    f = rng.standard_normal(200000).astype(np.float32) * np.float32(37.0)
    f = np.concatenate([f, rng.uniform(-1e-38, 1e-38, 1000).astype(np.float32)])
    assert np.array_equal(f32_to_bf16(f), _torch_bf16_bits(f))


def test_ties_round_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1 + 2^-7 -> rounds to 1.0 (even)
    tie_even = np.array([0x3F808000], np.uint32).view(np.float32)
    tie_odd = np.array([0x3F818000], np.uint32).view(np.float32)  # halfway above an odd mantissa
    assert f32_to_bf16(tie_even)[0] == 0x3F80
    assert f32_to_bf16(tie_odd)[0] == 0x3F82
    assert np.array_equal(f32_to_bf16(np.concatenate([tie_even, tie_odd])),
                          _torch_bf16_bits(np.concatenate([tie_even, tie_odd])))


def test_overflow_and_specials():
    big = np.array([3.4e38, -3.4e38, np.inf, -np.inf, 0.0, -0.0], np.float32)
    out = f32_to_bf16(big)
    assert out[0] == 0x7F80 and out[1] == 0xFF80  # rounds past max bf16 to +-Inf
    assert out[2] == 0x7F80 and out[3] == 0xFF80
    assert out[4] == 0x0000 and out[5] == 0x8000
    nan = np.array([0x7F800001], np.uint32).view(np.float32)  # payload only in low half
    assert np.isnan(bf16_to_f32(f32_to_bf16(nan)))[0]
