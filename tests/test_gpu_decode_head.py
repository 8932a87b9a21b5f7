"""The greedy decode tail, sc_decode_head_bf16 (final RMSNorm + lm_head + arg-max +
counter advance in one call), against the three calls it replaces
(sc_qmm_rmsnorm_bf16, sc_argmax_bf16, sc_add_i32) and against numpy's first-max
index on the logits it returns.

At batch 1 the lm_head GEMV selects the token in its epilogue: each workgroup maxes
its outputs' (value, ~index) keys into the workspace and the last workgroup to
finish writes the token, advances the counters and clears the workspace.  Rows
made identical in the weight (so their logits are equal and the largest) sit in
different workgroups, so the first-index rule is checked across workgroups.  At
batch 3 the separate kernels run.  Every call must leave the workspace zero, so
the calls run several times in a row on one workspace.
"""
import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.mlx_affine import quantize_bf16
from shardcompute_amd import _lib
from tests.gpu_util import dev_bf16, dev_u32, host_u16

pytestmark = pytest.mark.gpu


def _bf(rng, shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("M,N,K,bits,with_bias", [(1, 128256, 4096, 4, False), (1, 32000, 2048, 4, False),
                                                  (1, 1000, 512, 8, False), (1, 520, 576, 4, False),
                                                  (3, 5000, 1024, 4, False), (1, 4000, 1024, 4, True),
                                                  (2, 4000, 1024, 4, True)])
def test_decode_head_matches_separate_calls(device, M, N, K, bits, with_bias):
    rng = np.random.default_rng(N + K + M)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    tied = [N // 2 + 1, 5, N - 3]                      # equal rows, far apart: index 5 must win
    w[tied] = 0.05
    wq, s, b = quantize_bf16(w, 64, bits)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    # a linear bias is added to the rounded product; equal on the tied rows
    bias = None
    if with_bias:
        bh = _bf(rng, (N,), 0.5)
        bh[tied] = bh[5]
        bias = dev_bf16(bh)
    nw = dev_bf16(f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)))
    eps = 1e-5
    ws = torch.zeros(_lib.DECODE_HEAD_WORKSPACE_BYTES // 4, dtype=torch.int32, device="cuda")
    T = 5
    tokens = torch.full((M, T), -1, dtype=torch.int32, device="cuda")
    tokens_ref = tokens.clone()
    counters = torch.tensor([7, 2, 99], dtype=torch.int32, device="cuda")   # [length, step, untouched]
    counters_ref = counters.clone()
    ids = torch.empty(M, dtype=torch.int32, device="cuda")
    ids_ref = torch.empty_like(ids)
    picked = []
    for call in range(4):                               # steps 2, 3, 4, then 5 (past the token columns)
        print(f"decode_head M={M} N={N} K={K} W{bits} call {call}", flush=True)
        if call == 1:                                   # positive inputs: the tied rows hold the maximum
            x = f32_to_bf16((np.abs(rng.standard_normal((M, K))) + 0.5).astype(np.float32))
            nw_c = dev_bf16(f32_to_bf16(np.full(K, 1.0, np.float32)))
            r = None
        else:
            x, r, nw_c = _bf(rng, (M, K)), dev_bf16(_bf(rng, (M, K))), nw
        xd = dev_bf16(x)
        logits, xn = _lib.decode_head(xd, nw_c, eps, *W, ids, ws, residual=r, bias=bias, bits=bits,
                                      tokens=tokens, step=counters[1:], counters=counters, n_counters=2)
        y_ref, xn_ref = _lib.qmm_rmsnorm(xd, nw_c, eps, *W, residual=r, bias=bias, bits=bits)
        _lib.argmax(y_ref, ids=ids_ref, tokens=tokens_ref, step=counters_ref[1:])
        _lib.add_i32(counters_ref, 1, n=2)
        torch.cuda.synchronize()
        assert torch.equal(logits, y_ref) and torch.equal(xn, xn_ref)
        assert torch.equal(ids, ids_ref), (call, ids, ids_ref)
        assert torch.equal(tokens, tokens_ref) and torch.equal(counters, counters_ref)
        assert not ws.any(), "the workspace must be left zero"
        first = np.argmax(bf16_to_f32(host_u16(logits)), axis=-1)
        assert np.array_equal(ids.cpu().numpy(), first)
        if call == 1:
            assert (first == 5).all()
        picked.append(ids.cpu().numpy().copy())
    t = tokens.cpu().numpy()
    assert (t[:, :2] == -1).all()                       # columns before the first step stay untouched
    assert np.array_equal(t[:, 2:], np.stack(picked[:3], axis=1))
    assert counters.cpu().tolist() == [11, 6, 99]


def test_decode_head_rejects_bad_workspace(device):
    rng = np.random.default_rng(9)
    wq, s, b = quantize_bf16((rng.standard_normal((64, 512)) * 0.02).astype(np.float32), 64, 4)
    W = (dev_u32(wq), dev_bf16(s), dev_bf16(b))
    x = dev_bf16(_bf(rng, (1, 512)))
    nw = dev_bf16(f32_to_bf16(np.ones(512, np.float32)))
    ids = torch.empty(1, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="workspace"):
        _lib.decode_head(x, nw, 1e-5, *W, ids, torch.zeros(2, dtype=torch.int32, device="cuda"))
    ws = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.decode_head(x, nw, 1e-5, *W, ids, ws[1:])           # 4-byte aligned only
