"""The decode GEMV with a fused RMSNorm (+ residual) prologue and/or SwiGLU
epilogue against the standalone kernels around the plain product, and against
the oracle.

The norm prologue shares the arithmetic and row partition of the standalone
norm and keeps the product's tiling, and the GEMV sums split tiles in a fixed
order, so the norm-fused product agrees bit for bit.  The SwiGLU epilogue pairs
gate and up columns in one tile, which changes where the k-sum splits between
waves, so it agrees to rounding (a few elements move by a bf16 step of g or u); both are
checked against the
oracle at the linear tolerance.
"""
import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.decoder import rms_norm
from oracle.mlx_affine import quantize_bf16, quantized_matmul_f64
from shardcompute_amd import _lib
from tests.gpu_util import LINEAR_TOL, bf16_ulp_diff, dev_bf16, dev_u32, host_u16, max_abs_rel

pytestmark = pytest.mark.gpu


def _weights(rng, N, K, bits):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    return quantize_bf16(w, 64, bits)


def _bf(rng, shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("M,N,K,bits", [(1, 6144, 4096, 4), (3, 1000, 1024, 4), (8, 4096, 2048, 8),
                                        (1, 520, 576, 4), (16, 512, 1024, 4), (1, 128256, 4096, 4),
                                        (1, 1000, 512, 4), (1, 1000, 512, 8)])
def test_qmm_rmsnorm_matches_unfused(device, M, N, K, bits):
    rng = np.random.default_rng(M * 31 + N + K)
    wq, s, b = _weights(rng, N, K, bits)
    x, r = _bf(rng, (M, K)), _bf(rng, (M, K))
    nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    eps = 1e-5
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd, rd, nwd = dev_bf16(x), dev_bf16(r), dev_bf16(nw)
    print(f"qmm_rmsnorm M={M} N={N} K={K} W{bits}", flush=True)
    h = torch.empty_like(xd)
    y, xn = _lib.qmm_rmsnorm(xd, nwd, eps, *W, residual=rd, h_out=h, bits=bits)
    h2 = torch.empty_like(xd)
    xn2 = _lib.rms_norm(xd, nwd, eps, residual=rd, h_out=h2)
    y2 = _lib.qmm(xn2, *W, bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(xn, xn2) and torch.equal(y, y2)
    # without residual: no h_out written
    y3, xn3 = _lib.qmm_rmsnorm(xd, nwd, eps, *W, bits=bits)
    assert torch.equal(xn3, _lib.rms_norm(xd, nwd, eps))
    # against the oracle
    hr = f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(r))
    xnr = f32_to_bf16(rms_norm(bf16_to_f32(hr), nw, eps))
    ref = quantized_matmul_f64(xnr, wq, s, b, 64, bits)
    assert max_abs_rel(host_u16(y), ref) <= LINEAR_TOL


@pytest.mark.parametrize("M,I,K,bits,norm", [(1, 14336, 4096, 4, True), (1, 5632, 2048, 4, False),
                                              (3, 1024, 1024, 8, True), (12, 512, 1024, 4, True),
                                              (1, 2048, 576, 4, True), (1, 256, 512, 4, True),
                                              (1, 64, 512, 8, False), (16, 1792, 4096, 4, True),
                                              (32, 896, 2048, 8, False), (24, 1024, 3584, 4, False),
                                              (64, 1024, 1024, 4, False), (300, 1536, 2048, 8, True),
                                              (600, 2048, 4096, 4, False)])
def test_qmm_swiglu_matches_unfused(device, M, I, K, bits, norm):
    rng = np.random.default_rng(M * 7 + I + K)
    wq, s, b = _weights(rng, 2 * I, K, bits)
    x, r = _bf(rng, (M, K)), _bf(rng, (M, K))
    nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd, rd, nwd = dev_bf16(x), dev_bf16(r), dev_bf16(nw)
    print(f"qmm_swiglu M={M} I={I} K={K} W{bits} norm={norm}", flush=True)
    if norm:
        h = torch.empty_like(xd)
        act, xn = _lib.qmm_swiglu(xd, *W, norm_weight=nwd, residual=rd, h_out=h, bits=bits)
        h2 = torch.empty_like(xd)
        xn2 = _lib.rms_norm(xd, nwd, 1e-5, residual=rd, h_out=h2)
        assert torch.equal(h, h2) and torch.equal(xn, xn2)
    else:
        act, _ = _lib.qmm_swiglu(xd, *W, bits=bits)
        xn2 = xd
    act2 = _lib.silu_mul(_lib.qmm(xn2, *W, bits=bits))
    torch.cuda.synchronize()
    # the paired gate|up tiles split the k-sum between waves at other points than the
    # plain product's tiles, so the fp32 sums may round differently: a rare element
    # moves by a bf16 step of g or u (measured relative to the output's scale)
    a1, a2 = host_u16(act), host_u16(act2)
    assert max_abs_rel(a1, a2) <= 2e-3 and (bf16_ulp_diff(a1, a2) > 0).mean() < 0.02
    if M > 8:
        # 9-32 rows: the product's own split-K pass applies the gate, on the same sums;
        # more rows: the GEMM pairs gate and up columns in its tiles, same k order
        assert torch.equal(act, act2)
    xin = host_u16(xn2)
    gu = quantized_matmul_f64(xin, wq, s, b, 64, bits)
    g = bf16_to_f32(f32_to_bf16(gu[:, :I].astype(np.float32)))
    u = bf16_to_f32(f32_to_bf16(gu[:, I:].astype(np.float32)))
    ref = bf16_to_f32(f32_to_bf16((g / (np.float32(1) + np.exp(-g, dtype=np.float32))) * u))
    assert max_abs_rel(host_u16(act), ref) <= LINEAR_TOL


@pytest.mark.parametrize("M,bits", [(2048, 4), (2048, 8)])
def test_qmm_swiglu_prefill_shape_matches_unfused(device, M, bits):
    # the Llama-3-8B gate|up at a 2048-token prefill: wide tiles plus the 128-wide
    # launch for the partial last round, both pairing gate and up columns
    rng = np.random.default_rng(M + bits)
    I, K = 14336, 4096
    wq, s, b = _weights(rng, 2 * I, K, bits)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd = dev_bf16(_bf(rng, (M, K)))
    print(f"qmm_swiglu M={M} I={I} K={K} W{bits}", flush=True)
    act, _ = _lib.qmm_swiglu(xd, *W, bits=bits)
    act2 = _lib.silu_mul(_lib.qmm(xd, *W, bits=bits))
    torch.cuda.synchronize()
    assert torch.equal(act, act2)


@pytest.mark.parametrize("M,bits", [(9, 4), (16, 8), (32, 4), (200, 4), (1100, 8)])
def test_qmm_swiglu_batch_with_bias(device, M, bits):
    """Batched rows: silu(gate) * up from the GEMV's split-K pass (9-32 rows) or the
    GEMM's paired tiles (more), with a linear bias added to the rounded gate and up
    (as the plain product does), equals the plain product followed by silu_mul bit
    for bit."""
    rng = np.random.default_rng(M + 1000 * bits)
    I, K = 1536, 4096
    wq, s, b = _weights(rng, 2 * I, K, bits)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd = dev_bf16(_bf(rng, (M, K)))
    bias = dev_bf16(_bf(rng, (2 * I,), 0.1))
    print(f"qmm_swiglu bias M={M} W{bits}", flush=True)
    act, _ = _lib.qmm_swiglu(xd, *W, bias=bias, bits=bits)
    act2 = _lib.silu_mul(_lib.qmm(xd, *W, bias=bias, bits=bits))
    torch.cuda.synchronize()
    assert torch.equal(act, act2)


def test_gemv_is_reproducible(device):
    # tiles split between waves are summed in a fixed order: repeated launches agree
    rng = np.random.default_rng(3)
    for (N, K) in ((4096, 14336), (28672, 4096), (1000, 5120)):
        wq, s, b = _weights(rng, N, K, 4)
        W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
        x = dev_bf16(_bf(rng, (1, K)))
        ys = [_lib.qmm(x, *W) for _ in range(5)]
        torch.cuda.synchronize()
        assert all(torch.equal(ys[0], y) for y in ys[1:]), (N, K)


def test_fused_rejects_aliasing(device):
    rng = np.random.default_rng(4)
    wq, s, b = _weights(rng, 64, 512, 4)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    x, r = dev_bf16(_bf(rng, (1, 512))), dev_bf16(_bf(rng, (1, 512)))
    nw = dev_bf16(f32_to_bf16(np.ones(512, np.float32)))
    with pytest.raises(RuntimeError, match="overlap"):
        _lib.qmm_rmsnorm(x, nw, 1e-5, *W, residual=r, h_out=x)
    with pytest.raises(RuntimeError, match="overlap"):
        _lib.qmm_rmsnorm(x, nw, 1e-5, *W, residual=r, xn_out=r)


@pytest.mark.parametrize("M,N,K,bits,with_bias", [(1, 4096, 4096, 4, False), (8, 4096, 14336, 4, True),
                                                  (16, 4096, 4096, 4, False), (16, 4096, 14336, 4, True),
                                                  (32, 8192, 1024, 4, False), (32, 8192, 3584, 8, True),
                                                  (24, 2048, 5632, 4, False), (64, 4096, 4096, 4, True),
                                                  (300, 2048, 2048, 8, False), (12, 16384, 1024, 4, False)])
def test_qmm_add_rmsnorm_matches_unfused(device, M, N, K, bits, with_bias):
    """The projection before a residual add and RMSNorm (o_proj, down_proj) with its
    split-K pass folded into the norm's: h and xn bit for bit the plain product (its
    own split-K pass, bias after rounding) followed by the standalone norm with that
    residual, on every kernel the product takes (decode GEMV, band kernel with and
    without K splits, GEMM); xn against the oracle."""
    rng = np.random.default_rng(M * 13 + N + K + bits)
    wq, s, b = _weights(rng, N, K, bits)
    x, r = _bf(rng, (M, K)), _bf(rng, (M, N), 4.0)
    nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(N)).astype(np.float32))
    bias = _bf(rng, (N,), 0.5) if with_bias else None
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd, rd, nwd = dev_bf16(x), dev_bf16(r), dev_bf16(nw)
    bd = dev_bf16(bias) if with_bias else None
    print(f"qmm_add_rmsnorm M={M} N={N} K={K} W{bits} bias={with_bias}", flush=True)
    h, xn = _lib.qmm_add_rmsnorm(xd, *W, rd, nwd, 1e-5, bias=bd, bits=bits)
    y = _lib.qmm(xd, *W, bias=bd, bits=bits)
    h2 = torch.empty_like(y)
    xn2 = _lib.rms_norm(y, nwd, 1e-5, residual=rd, h_out=h2)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(xn, xn2)
    # the same buffers again (every output element rewritten; nothing carried over)
    h.fill_(0)
    xn.fill_(0)
    _lib.qmm_add_rmsnorm(xd, *W, rd, nwd, 1e-5, bias=bd, bits=bits, h_out=h, xn_out=xn)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(xn, xn2)
    ref = quantized_matmul_f64(x, wq, s, b, 64, bits)
    yr = bf16_to_f32(f32_to_bf16(ref.astype(np.float32)))
    if with_bias:
        yr = bf16_to_f32(f32_to_bf16(yr + bf16_to_f32(bias)[None]))
    hr = f32_to_bf16(yr + bf16_to_f32(r))
    xnr = rms_norm(bf16_to_f32(hr), nw, 1e-5)
    assert max_abs_rel(host_u16(xn), xnr) <= LINEAR_TOL


def test_qmm_add_rmsnorm_rejects_overlap(device):
    rng = np.random.default_rng(5)
    wq, s, b = _weights(rng, 1024, 1024, 4)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    xd, rd = dev_bf16(_bf(rng, (16, 1024))), dev_bf16(_bf(rng, (16, 1024)))
    nwd = dev_bf16(f32_to_bf16(np.ones(1024, np.float32)))
    with pytest.raises(RuntimeError, match="overlap"):
        _lib.qmm_add_rmsnorm(xd, *W, rd, nwd, 1e-5, h_out=rd)
    with pytest.raises(RuntimeError, match="overlap"):
        out = torch.empty_like(rd)
        _lib.qmm_add_rmsnorm(xd, *W, rd, nwd, 1e-5, h_out=out, xn_out=out)
