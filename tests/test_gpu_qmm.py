"""Parity of the HIP quantized matmul (both kernels) with the oracle, through the C-ABI.

Tolerance: max|y - ref| / max|ref| <= 1e-2 (bf16 output, fp32 accumulation);
the kernels actually land within a couple of bf16 steps of the fp64 oracle,
which the tighter informational checks below also assert.
"""
import os

import numpy as np
import pytest
import torch

from oracle import cref
from oracle.bf16 import f32_to_bf16
from oracle.mlx_affine import quantize_bf16, quantized_matmul_bf16, quantized_matmul_f64
from shardcompute_amd import _lib
from tests.gpu_util import LINEAR_TOL, bf16_ulp_diff, dev_bf16, dev_u32, host_u16, max_abs_rel

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _case(rng, M, K, N, bits, with_bias):
    x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, s, b = quantize_bf16(w, 64, bits)
    bias = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1) if with_bias else None
    return x, wq, s, b, bias


def _run(x, wq, s, b, bias, bits, path):
    y = _lib.qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b),
                 None if bias is None else dev_bf16(bias), bits=bits, path=path)
    torch.cuda.synchronize()
    return host_u16(y)


def _paths(M):
    return [_lib.PATH_GEMV, _lib.PATH_GEMM] if M <= 32 else [_lib.PATH_GEMM]


def test_golden_fixtures_both_kernels(device):
    z = np.load(os.path.join(GOLD, "qmm_cases.npz"), allow_pickle=False)
    for i in range(int(z["n_cases"])):
        p = f"c{i}_"
        M, K, N, bits, has_bias = z[p + "meta"].tolist()
        bias = z[p + "bias"] if has_bias else None
        for path in _paths(M):
            print(f"golden case {i} M={M} K={K} N={N} bits={bits} path={path}", flush=True)
            y = _run(z[p + "x"], z[p + "wq"], z[p + "s"], z[p + "b"], bias, bits, path)
            assert max_abs_rel(y, z[p + "y"]) <= LINEAR_TOL
            assert bf16_ulp_diff(y, z[p + "y"]).max() <= 2, (i, path)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 9, 16, 17, 31, 32])
def test_gemv_random_shapes(device, bits, M):
    rng = np.random.default_rng(100 + M + bits)
    for K, N in [(64, 1), (576, 33), (1024, 257), (4096, 96), (2048, 1000)]:
        with_bias = (N % 2) == 1
        x, wq, s, b, bias = _case(rng, M, K, N, bits, with_bias)
        print(f"gemv M={M} K={K} N={N} bits={bits}", flush=True)
        y = _run(x, wq, s, b, bias, bits, _lib.PATH_GEMV)
        ref = quantized_matmul_bf16(x, wq, s, b, bias, 64, bits)
        assert max_abs_rel(y, ref) <= LINEAR_TOL
        assert bf16_ulp_diff(y, ref).max() <= 2


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 33, 64, 127, 128, 130, 257])
def test_gemm_random_shapes(device, bits, M):
    rng = np.random.default_rng(200 + M + bits)
    for K, N in [(64, 5), (576, 130), (1024, 256), (2048, 300)]:
        x, wq, s, b, bias = _case(rng, M, K, N, bits, N % 2 == 0)
        print(f"gemm M={M} K={K} N={N} bits={bits}", flush=True)
        y = _run(x, wq, s, b, bias, bits, _lib.PATH_GEMM)
        ref = quantized_matmul_bf16(x, wq, s, b, bias, 64, bits)
        assert max_abs_rel(y, ref) <= LINEAR_TOL
        assert bf16_ulp_diff(y, ref).max() <= 2


def test_split_k_is_deterministic_and_reusable(device):
    # small N forces split-K; repeated calls (scratch reuse, counters reset) give identical bits
    rng = np.random.default_rng(7)
    x, wq, s, b, bias = _case(rng, 4, 8192, 64, 4, True)
    ys = [_run(x, wq, s, b, bias, 4, _lib.PATH_GEMV) for _ in range(3)]
    assert all(np.array_equal(ys[0], y) for y in ys[1:])
    ref = quantized_matmul_bf16(x, wq, s, b, bias, 64, 4)
    assert max_abs_rel(ys[0], ref) <= LINEAR_TOL
    # a larger split-K shape after a smaller one grows the scratch
    x2, wq2, s2, b2, _ = _case(rng, 32, 14336, 128, 8, False)
    y2 = _run(x2, wq2, s2, b2, None, 8, _lib.PATH_GEMV)
    assert max_abs_rel(y2, quantized_matmul_bf16(x2, wq2, s2, b2, None, 64, 8)) <= LINEAR_TOL


SWEEP = [(2048, 2560), (2048, 5632), (5632, 2048), (4096, 6144), (4096, 14336), (14336, 4096)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,N", SWEEP)
def test_full_size_decode_shapes_vs_c_oracle(device, bits, K, N):
    """The standalone sweep's (K, N) pairs at decode batch sizes, all outputs checked."""
    if not cref.available():
        cref.build()
    rng = np.random.default_rng(K + N + bits)
    _, wq, s, b, _ = _case(rng, 1, K, N, bits, False)
    for M in (1, 8, 32):
        x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
        print(f"full-size gemv K={K} N={N} bits={bits} M={M}", flush=True)
        y = _run(x, wq, s, b, None, bits, _lib.PATH_AUTO)
        ref = cref.qmm_bf16(x, wq, s, b, None, 64, bits)
        assert max_abs_rel(y, ref) <= LINEAR_TOL
        assert bf16_ulp_diff(y, ref).max() <= 2


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,N", SWEEP)
def test_full_size_prefill_shapes(device, bits, K, N):
    """M = 512 / 2048: 24 sampled rows against the fp64 oracle, every row against
    the independent GEMV kernel (row m of a batched product equals the product
    of row m alone)."""
    rng = np.random.default_rng(K * 3 + N + bits)
    _, wq, s, b, _ = _case(rng, 1, K, N, bits, False)
    for M in (512, 2048):
        x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
        print(f"full-size gemm K={K} N={N} bits={bits} M={M}", flush=True)
        y = _run(x, wq, s, b, None, bits, _lib.PATH_AUTO)
        rows = np.sort(rng.choice(M, 24, replace=False))
        ref = f32_to_bf16(quantized_matmul_f64(x[rows], wq, s, b, 64, bits).astype(np.float32))
        assert max_abs_rel(y[rows], ref) <= LINEAR_TOL
        assert bf16_ulp_diff(y[rows], ref).max() <= 2
        for r0 in range(0, M, 32):
            yg = _run(x[r0:r0 + 32], wq, s, b, None, bits, _lib.PATH_GEMV)
            assert bf16_ulp_diff(y[r0:r0 + 32], yg).max() <= 2


def test_linearity_in_x(device):
    rng = np.random.default_rng(9)
    x1, wq, s, b, _ = _case(rng, 8, 4096, 512, 4, False)
    x2 = f32_to_bf16(rng.standard_normal((8, 4096)).astype(np.float32))
    t1, t2 = dev_bf16(x1), dev_bf16(x2)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    y1 = _lib.qmm(t1, *W).float()
    y2 = _lib.qmm(t2, *W).float()
    y12 = _lib.qmm((t1.float() + t2.float()).bfloat16(), *W).float()
    err = (y12 - (y1 + y2)).abs().max() / (y1 + y2).abs().max()
    assert err.item() < 2e-2


def test_leading_dims_and_errors(device):
    rng = np.random.default_rng(10)
    x, wq, s, b, _ = _case(rng, 6, 256, 64, 4, False)
    xt = dev_bf16(x).reshape(2, 3, 256)
    y = _lib.qmm(xt, dev_u32(wq), dev_bf16(s), dev_bf16(b))
    assert tuple(y.shape) == (2, 3, 64)
    ref = quantized_matmul_bf16(x, wq, s, b, None, 64, 4)
    assert max_abs_rel(host_u16(y.reshape(6, 64)), ref) <= LINEAR_TOL
    with pytest.raises(ValueError):
        _lib.qmm(dev_bf16(x[:, :192]), dev_u32(wq), dev_bf16(s), dev_bf16(b))
    with pytest.raises(RuntimeError):
        # misaligned x (offset by one element) is rejected by the library
        buf = torch.empty(6 * 256 + 1, dtype=torch.bfloat16, device="cuda")
        xm = buf[1:].view(6, 256)
        _lib.qmm(xm, dev_u32(wq), dev_bf16(s), dev_bf16(b))
    with pytest.raises(RuntimeError):
        _lib.qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), bits=4, group_size=32)
