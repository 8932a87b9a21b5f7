"""The middle-band quantized product (9-256 rows, sc_qmm_bf16_band / SC_QMM_PATH_BAND)
against the oracle, through the C-ABI.

The band kernel rounds every dequantized weight s*q + b to bf16 before the MFMA, as the
GEMM does, so it gets the GEMM's bars: max|y - ref| / max|ref| <= 1e-2 and
mean|y - ref| / max|ref| <= 2e-3, with the reference layer's order (bf16 product, then
the bias added and rounded again).  Every plan (4- or 8-wave workgroups, any K split)
must meet them; repeated launches of one plan are bit-identical (the split-K pass sums
in split order).
"""
import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.mlx_affine import quantize_bf16, quantized_matmul_bf16
from shardcompute_amd import _lib
from tests.gpu_util import LINEAR_TOL, dev_bf16, dev_u32, host_u16, max_abs_rel

pytestmark = pytest.mark.gpu


def _case(rng, M, K, N, bits, with_bias):
    x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, s, b = quantize_bf16(w, 64, bits)
    bias = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1) if with_bias else None
    return x, wq, s, b, bias


def _band(x, wq, s, b, bias, bits, plan):
    y = _lib.qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), None if bias is None else dev_bf16(bias),
                 bits=bits, band_plan=plan)
    torch.cuda.synchronize()
    return host_u16(y)


def _assert_gemm_bars(y, ref):
    assert max_abs_rel(y, ref) <= LINEAR_TOL
    yf, rf = bf16_to_f32(y).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    assert np.mean(np.abs(yf - rf)) / np.max(np.abs(rf)) <= 2e-3


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [9, 16, 32, 33, 64, 100, 128, 129, 200, 256])
def test_band_random_shapes(device, bits, M):
    rng = np.random.default_rng(300 + M + bits)
    # N not a multiple of the 32-row wave tile, one row, and K of 1 to 28 scale blocks
    for K, N in [(512, 1), (1024, 257), (2048, 300), (4096, 96), (3584, 520), (14336, 40)]:
        x, wq, s, b, bias = _case(rng, M, K, N, bits, N % 2 == 0)
        ref = quantized_matmul_bf16(x, wq, s, b, bias, 64, bits)
        for plan in [(0, 0), (4, 1), (8, 1), (8, 3), (4, 5)]:
            print(f"band M={M} K={K} N={N} W{bits} plan={plan}", flush=True)
            _assert_gemm_bars(_band(x, wq, s, b, bias, bits, plan), ref)


def test_band_every_split_count(device):
    # K = 8192: 16 scale blocks, split 1 .. 16 ways (uneven last splits included)
    rng = np.random.default_rng(11)
    x, wq, s, b, bias = _case(rng, 32, 8192, 160, 4, True)
    ref = quantized_matmul_bf16(x, wq, s, b, bias, 64, 4)
    for ks in range(1, 17):
        print(f"band ksplit={ks}", flush=True)
        _assert_gemm_bars(_band(x, wq, s, b, bias, 4, (4, ks)), ref)


def test_band_is_reproducible(device):
    rng = np.random.default_rng(12)
    x, wq, s, b, bias = _case(rng, 64, 4096, 1000, 4, False)
    for plan in [(8, 1), (4, 4)]:
        ys = [_band(x, wq, s, b, bias, 4, plan) for _ in range(3)]
        assert all(np.array_equal(ys[0], y) for y in ys[1:]), plan


def test_band_refuses_what_it_does_not_take(device):
    rng = np.random.default_rng(13)
    x, wq, s, b, _ = _case(rng, 16, 576, 64, 4, False)      # K not a multiple of 512
    with pytest.raises(RuntimeError, match="not taken"):
        _band(x, wq, s, b, None, 4, (0, 0))
    x, wq, s, b, _ = _case(rng, 257, 512, 64, 4, False)      # more than 256 rows
    with pytest.raises(RuntimeError, match="not taken"):
        _band(x, wq, s, b, None, 4, (0, 0))
    # the automatic path falls back to the GEMM for the first
    x, wq, s, b, _ = _case(rng, 40, 576, 64, 4, False)
    y = _lib.qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), bits=4)
    torch.cuda.synchronize()
    _assert_gemm_bars(host_u16(y), quantized_matmul_bf16(x, wq, s, b, None, 64, 4))


@pytest.mark.parametrize("bits", [4, 8])
def test_band_lm_head_64_positions(device, bits):
    """The vocab-sharded lm_head over 64 last positions (rank 0 of 2 of a 128256-token
    vocabulary: [64128, 4096] at W4/W8), on the automatic path: every output column of
    a sample of 640 against the oracle, the rest against the tiled GEMM."""
    rng = np.random.default_rng(14 + bits)
    M, K, N = 64, 4096, 64128
    x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    wq, s, b = [], [], []
    for r0 in range(0, N, 8192):                      # quantize in slices (memory)
        w = (rng.standard_normal((min(8192, N - r0), K)) * 0.02).astype(np.float32)
        q = quantize_bf16(w, 64, bits)
        wq.append(q[0]), s.append(q[1]), b.append(q[2])
    wq, s, b = np.concatenate(wq), np.concatenate(s), np.concatenate(b)
    xd, W = dev_bf16(x), (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    print(f"band lm_head M={M} K={K} N={N} W{bits}", flush=True)
    y = _lib.qmm(xd, *W, bits=bits)
    y_gemm = _lib.qmm(xd, *W, bits=bits, path=_lib.PATH_GEMM)
    torch.cuda.synchronize()
    yh = host_u16(y)
    cols = np.sort(rng.choice(N, size=640, replace=False))
    ref = quantized_matmul_bf16(x, wq[cols], s[cols], b[cols], None, 64, bits)
    _assert_gemm_bars(yh[:, cols], ref)
    assert max_abs_rel(yh, host_u16(y_gemm)) <= LINEAR_TOL
