"""The oracle still reproduces every committed golden fixture bit for bit."""
import os

import numpy as np
import pytest

from oracle.gather import qembed_gather_bf16, vocab_gather_bf16
from oracle.mlx_affine import quantize_bf16, quantized_matmul_bf16

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_qmm_fixtures():
    z = _load("qmm_cases.npz")
    for i in range(int(z["n_cases"])):
        p = f"c{i}_"
        M, K, N, bits, has_bias = z[p + "meta"].tolist()
        bias = z[p + "bias"] if has_bias else None
        y = quantized_matmul_bf16(z[p + "x"], z[p + "wq"], z[p + "s"], z[p + "b"], bias, 64, bits)
        assert y.shape == (M, N)
        assert np.array_equal(y, z[p + "y"]), f"case {i}"


def test_gather_fixtures():
    z = _load("gather_cases.npz")
    assert np.array_equal(vocab_gather_bf16(z["ids"], z["table"], int(z["start"])), z["out"])
    assert np.array_equal(vocab_gather_bf16(z["vids"], z["vtable"], int(z["vstart"])), z["vout"])
    assert np.array_equal(vocab_gather_bf16(z["oids"], z["otable"], int(z["ostart"])), z["oout"])


@pytest.mark.parametrize("bits", [4, 8])
def test_qembed_fixtures(bits):
    z = _load("qembed_cases.npz")
    p = f"w{bits}_"
    got = qembed_gather_bf16(z[p + "ids"], z[p + "wq"], z[p + "s"], z[p + "b"], int(z["start"]), 64, bits)
    assert np.array_equal(got, z[p + "out"])


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_fixtures(bits):
    z = _load("quantize_cases.npz")
    wq, s, b = quantize_bf16(z["w"], 64, bits)
    assert np.array_equal(wq, z[f"wq{bits}"])
    assert np.array_equal(s, z[f"s{bits}"]) and np.array_equal(b, z[f"b{bits}"])
