"""Parity of the HIP quantized matmul (both kernels) with the oracle, through the C-ABI.

Tolerance: max|y - ref| / max|ref| <= 1e-2 (bf16 output, fp32 accumulation).
Tighter checks per kernel:
* GEMV keeps the codes exact (bf16 128 + q) and applies scale and bias per
  group in fp32: |y - ref| <= 2 bf16 steps + 1e-5 * max|ref|.  The steps are
  taken at the larger of |ref| and |ref - bias|, because the layer rounds the
  matmul to bf16 before adding the linear bias (one step of the pre-bias value
  can be many steps of a result the bias nearly cancels); the second term is
  fp32 accumulation noise, visible only on near-zero outputs.
* GEMM rounds every dequantized weight s*q + b to bf16 before the MFMA (half a
  bf16 step, 2^-9 relative, per weight), so its mean error is bounded instead:
  mean|y - ref| / max|ref| <= 2e-3.
"""
import os

import numpy as np
import pytest
import torch

from oracle import cref
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.mlx_affine import quantize_bf16, quantized_matmul_bf16, quantized_matmul_f64
from shardcompute_amd import _lib
from tests.gpu_util import LINEAR_TOL, dev_bf16, dev_u32, host_u16, max_abs_rel

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


def assert_close(y, ref, path, bias=None):
    assert max_abs_rel(y, ref) <= LINEAR_TOL
    yf, rf = bf16_to_f32(y).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    if path == _lib.PATH_GEMV:
        mag = np.abs(rf)
        if bias is not None:
            mag = np.maximum(mag, np.abs(rf - bf16_to_f32(bias).astype(np.float64)[None, :]))
        _, e = np.frexp(mag)
        ulp = np.ldexp(1.0, e - 8)
        err = np.abs(yf - rf)
        bound = 2 * ulp + 1e-5 * np.max(np.abs(rf))
        bad = np.argwhere(err > bound)
        assert bad.size == 0, f"{len(bad)} outputs off, first {bad[0]}: y={yf[tuple(bad[0])]} ref={rf[tuple(bad[0])]}"
    else:
        assert np.mean(np.abs(yf - rf)) / np.max(np.abs(rf)) <= 2e-3


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
            assert_close(y, z[p + "y"], path, bias)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 9, 16, 17, 31, 32])
def test_gemv_random_shapes(device, bits, M):
    rng = np.random.default_rng(100 + M + bits)
    # (6656, 48): 13 (W4) / 26 (W8) K splits at 9-32 rows, so the split-K pass sums
    # blocks of eight and four partials and single ones
    for K, N in [(64, 1), (576, 33), (1024, 257), (4096, 96), (2048, 1000), (512, 71), (14336, 40), (6656, 48)]:
        with_bias = (N % 2) == 1
        x, wq, s, b, bias = _case(rng, M, K, N, bits, with_bias)
        print(f"gemv M={M} K={K} N={N} bits={bits}", flush=True)
        y = _run(x, wq, s, b, bias, bits, _lib.PATH_GEMV)
        assert_close(y, quantized_matmul_bf16(x, wq, s, b, bias, 64, bits), _lib.PATH_GEMV, bias)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 33, 64, 127, 128, 130, 257])
def test_gemm_random_shapes(device, bits, M):
    rng = np.random.default_rng(200 + M + bits)
    for K, N in [(64, 5), (576, 130), (1024, 256), (2048, 300)]:
        x, wq, s, b, bias = _case(rng, M, K, N, bits, N % 2 == 0)
        print(f"gemm M={M} K={K} N={N} bits={bits}", flush=True)
        y = _run(x, wq, s, b, bias, bits, _lib.PATH_GEMM)
        assert_close(y, quantized_matmul_bf16(x, wq, s, b, bias, 64, bits), _lib.PATH_GEMM)


def test_split_k_is_deterministic_and_reusable(device):
    # small N forces split-K; repeated calls (scratch reuse, counters reset) give identical bits
    rng = np.random.default_rng(7)
    x, wq, s, b, bias = _case(rng, 4, 8192, 64, 4, True)
    ys = [_run(x, wq, s, b, bias, 4, _lib.PATH_GEMV) for _ in range(3)]
    assert all(np.array_equal(ys[0], y) for y in ys[1:])
    assert_close(ys[0], quantized_matmul_bf16(x, wq, s, b, bias, 64, 4), _lib.PATH_GEMV, bias)
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
        assert_close(y, cref.qmm_bf16(x, wq, s, b, None, 64, bits), _lib.PATH_GEMV)


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
        assert_close(y[rows], ref, _lib.PATH_GEMM)
        W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
        xd = dev_bf16(x)
        yg = torch.cat([_lib.qmm(xd[r0:r0 + 32], *W, bits=bits, path=_lib.PATH_GEMV) for r0 in range(0, M, 32)])
        assert max_abs_rel(y, host_u16(yg)) <= LINEAR_TOL


@pytest.mark.parametrize("M,K,N,bits,with_bias", [(256, 64, 153600, 4, True), (256, 64, 153600, 8, True),
                                                     (2048, 4096, 28672, 4, False)])
def test_prefill_split_launch(device, M, K, N, bits, with_bias):
    """Wide tiles that leave a partial last round over the CUs run as two launches
    (the last round's columns with 128-wide tiles): every output, across the column
    split and with the bias on both sides of it, against the GEMV on 32-row blocks,
    and sampled rows against the fp64 oracle."""
    rng = np.random.default_rng(M + K + N + bits)
    x, wq, s, b, bias = _case(rng, M, K, N, bits, with_bias)
    print(f"gemm split M={M} K={K} N={N} bits={bits} bias={with_bias}", flush=True)
    y = _run(x, wq, s, b, bias, bits, _lib.PATH_GEMM)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd, bd = dev_bf16(x), None if bias is None else dev_bf16(bias)
    yg = torch.cat([_lib.qmm(xd[r0:r0 + 32], *W, bd, bits=bits, path=_lib.PATH_GEMV) for r0 in range(0, M, 32)])
    assert max_abs_rel(y, host_u16(yg)) <= LINEAR_TOL
    rows = np.sort(rng.choice(M, 8, replace=False))
    ref = f32_to_bf16((quantized_matmul_f64(x[rows], wq, s, b, 64, bits)
                       + (0 if bias is None else bf16_to_f32(bias).astype(np.float64))).astype(np.float32))
    assert max_abs_rel(y[rows], ref) <= LINEAR_TOL


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
    with pytest.raises((RuntimeError, ValueError)):
        _lib.qmm(dev_bf16(x), dev_u32(wq), dev_bf16(s), dev_bf16(b), bits=4, group_size=32)


# (K, N, M, bits): the vocab-parallel lm_head of the world_size=2 rank-0 share
# (64128 rows, the last positions of 64 sequences), and the Llama-3-70B rank-0
# shard of world_size=8 (q|k|v 8192 -> 1024 + 2 * 128, o 1024 -> 8192, gate|up
# 8192 -> 2 * 3584, down 3584 -> 8192) at batch-32 decode and 1024-token prefill
CONFIG_SHAPES = [(4096, 64128, 64, 4)] + [(K, N, M, bits) for (K, N) in
                                           [(8192, 1280), (1024, 8192), (8192, 7168), (3584, 8192)]
                                           for M in (32, 1024) for bits in (4, 8)]


@pytest.mark.parametrize("K,N,M,bits", CONFIG_SHAPES)
def test_config_shard_shapes(device, K, N, M, bits):
    """Sampled rows against the fp64 oracle, every row against the GEMV kernel."""
    rng = np.random.default_rng(K + 7 * N + M + bits)
    _, wq, s, b, _ = _case(rng, 1, K, N, bits, False)
    x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    print(f"config shape K={K} N={N} M={M} bits={bits}", flush=True)
    y = _run(x, wq, s, b, None, bits, _lib.PATH_AUTO)
    rows = np.sort(rng.choice(M, min(M, 16), replace=False))
    ref = f32_to_bf16(quantized_matmul_f64(x[rows], wq, s, b, 64, bits).astype(np.float32))
    assert_close(y[rows], ref, _lib.PATH_GEMV if M <= 32 else _lib.PATH_GEMM)
    if M > 32:
        W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
        xd = dev_bf16(x)
        yg = torch.cat([_lib.qmm(xd[r0:r0 + 32], *W, bits=bits, path=_lib.PATH_GEMV) for r0 in range(0, M, 32)])
        assert max_abs_rel(y, host_u16(yg)) <= LINEAR_TOL
