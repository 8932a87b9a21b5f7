"""sc_qmm_bf16_noalloc, the allocation-free quantized product, against sc_qmm_bf16.

Both entry points are called through the C-ABI (ctypes) on the same inputs; the
outputs must be identical bit for bit (same kernels; only where the split-K
partials live differs).  Covered:

* shapes on every kernel path: the batch-1 / <= 8-row GEMV, the 9-32-row
  split-K GEMV and the 33-160-row band kernel (the paths that use the scratch
  array: small N, large K, as the 70B shard's k/v projection), and the MFMA GEMM;
* two calls in a row, the second with a smaller input (the array keeps the
  first call's partials; nothing may leak into the second);
* a fresh split-K shape captured in a HIP graph at its first call (the
  library-owned scratch would allocate and synchronise there), replayed three
  times with eager work between replays, each replay equal to the eager result;
  and the same in a fresh process whose very first library product is the captured
  no-alloc call (the scratch array's address is looked up under capture there);
* a shape whose partials exceed SC_QMM_NOALLOC_SCRATCH_BYTES runs on a kernel that
  needs no scratch: within 1e-2 of sc_qmm_bf16's result and of the oracle.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from shardcompute_amd import _lib

pytestmark = pytest.mark.gpu


def _weights(g, N, K, bits):
    return _lib.quantize(torch.randn((N, K), generator=g, device="cuda").mul_(0.02), bits=bits)


def _call(entry, x, wq, s, b, bias, y, bits):
    lib = _lib.load()
    M, K = x.shape
    N = wq.shape[0]
    fn = getattr(lib, entry)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = fn(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(wq.data_ptr()), ctypes.c_void_p(s.data_ptr()),
            ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(bias.data_ptr()) if bias is not None else None,
            ctypes.c_void_p(y.data_ptr()), M, N, K, bits, 64, st)
    return rc


def _pair(g, M, N, K, bits, with_bias):
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    wq, s, b = _weights(g, N, K, bits)
    bias = torch.randn(N, generator=g, device="cuda").to(torch.bfloat16) if with_bias else None
    y_ref = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    y_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert _call("sc_qmm_bf16", x, wq, s, b, bias, y_ref, bits) == 0
    rc = _call("sc_qmm_bf16_noalloc", x, wq, s, b, bias, y_na, bits)
    assert rc == 0, _lib.load().sc_last_error().decode()
    torch.cuda.synchronize()
    return y_ref, y_na


# (M, N, K): split-K GEMV (9-32 rows, small N), batch-1 GEMV, 8-row GEMV, the band
# kernel with K splits (33-160 rows), the GEMM; then the smaller second call of each pair
PAIRS = [((32, 128, 8192), (12, 128, 4096)), ((24, 1024, 8192), (9, 256, 2048)),
         ((1, 4096, 4096), (1, 1024, 2048)), ((8, 2048, 4096), (3, 512, 1024)),
         ((64, 512, 2048), (40, 256, 1024)), ((200, 256, 1024), (170, 128, 512))]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_equals_qmm_two_calls(device, bits, first, second):
    g = torch.Generator(device="cuda")
    g.manual_seed(hash((bits,) + first) % (2 ** 31))
    for i, (M, N, K) in enumerate((first, second)):
        print(f"noalloc bits={bits} call {i}: M={M} N={N} K={K}", flush=True)
        y_ref, y_na = _pair(g, M, N, K, bits, with_bias=(i == 1))
        assert torch.equal(y_ref, y_na), f"call {i} differs at M={M} N={N} K={K}"


def test_noalloc_under_graph_capture(device):
    # a split-K shape not used before in this process: sc_qmm_bf16 would allocate its
    # scratch (and synchronise) here; the no-alloc entry point captures as is
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    M, N, K, bits = 20, 64, 14336, 4
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    wq, s, b = _weights(g, N, K, bits)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call("sc_qmm_bf16_noalloc", x, wq, s, b, None, y, bits)
    assert rc == 0, _lib.load().sc_last_error().decode()
    ref = torch.empty_like(y)
    assert _call("sc_qmm_bf16", x, wq, s, b, None, ref, bits) == 0
    torch.cuda.synchronize()
    for r in range(3):
        y.fill_(float("nan"))
        # eager work between replays that reuses the scratch array with other partials
        other = torch.empty((12, 128), dtype=torch.bfloat16, device="cuda")
        xo = torch.randn((12, 8192), generator=g, device="cuda").to(torch.bfloat16)
        wo = _weights(g, 128, 8192, bits)
        assert _call("sc_qmm_bf16_noalloc", xo, *wo, None, other, bits) == 0
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {r} differs from the eager product"


def test_noalloc_oversized_scratch_falls_back(device):
    # 32 rows with K = 65536: the 9-32-row GEMV splits K 32 ways, so its partials are
    # 32 * 32 * 2048 floats = 8 MiB, above the 4 MiB array: the no-alloc entry point
    # takes a kernel without split-K scratch instead of refusing
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    M, N, K, bits = 32, 2048, 65536, 4
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    wq, s, b = _weights(g, N, K, bits)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    rc = _call("sc_qmm_bf16_noalloc", x, wq, s, b, None, y, bits)
    assert rc == 0, _lib.load().sc_last_error().decode()
    ref = torch.empty_like(y)
    assert _call("sc_qmm_bf16", x, wq, s, b, None, ref, bits) == 0
    torch.cuda.synchronize()
    from oracle.mlx_affine import quantized_matmul_f64
    from tests.gpu_util import host_u16, host_u32, max_abs_rel
    assert max_abs_rel(host_u16(y), host_u16(ref).astype(np.uint16)) <= 1e-2
    r = quantized_matmul_f64(host_u16(x[:2]), host_u32(wq), host_u16(s), host_u16(b), bits=bits)
    assert np.isfinite(r).all()
    assert max_abs_rel(host_u16(y[:2]), r) <= 1e-2
    assert max_abs_rel(host_u16(ref[:2]), r) <= 1e-2


_FIRST_CALL_CAPTURED = r"""
import ctypes, sys, torch
sys.path.insert(0, sys.argv[1])
from shardcompute_amd import _lib
lib = _lib.load()
g = torch.Generator(device="cuda"); g.manual_seed(9)
M, N, K, bits = 20, 64, 14336, 4
x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
wq, s, b = _lib.quantize(torch.randn((N, K), generator=g, device="cuda").mul_(0.02), bits=bits)
y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
ref = torch.empty_like(y)
P = ctypes.c_void_p
def call(entry, out):
    st = P(torch.cuda.current_stream().cuda_stream)
    return getattr(lib, entry)(P(x.data_ptr()), P(wq.data_ptr()), P(s.data_ptr()), P(b.data_ptr()), None,
                               P(out.data_ptr()), M, N, K, bits, 64, st)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = call("sc_qmm_bf16_noalloc", y)          # the process's first product: address lookup under capture
assert rc == 0, lib.sc_last_error().decode()
assert call("sc_qmm_bf16", ref) == 0
torch.cuda.synchronize()
for r in range(3):
    y.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref), f"replay {r}"
print("first captured call ok", flush=True)
"""


def test_noalloc_first_call_under_capture_fresh_process(device):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("fresh process: first no-alloc call under graph capture", flush=True)
    p = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                       timeout=240, cwd=root)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-4000:]
    assert "first captured call ok" in p.stdout
