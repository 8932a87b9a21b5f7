"""ctypes binding of libshardcompute_hip.so over torch-ROCm tensors.

Every wrapper checks shapes/dtypes on the host, allocates its output with torch
on the input's device, passes raw device pointers and torch's current HIP
stream, and raises ``RuntimeError`` with the library's message when the C-ABI
returns a non-zero status.  There is no CPU fallback: if the library is not
built, or a tensor is not on a GPU, the call raises.
"""
import ctypes
import os
import threading

import torch

from .build import LIB_PATH

ABI_VERSION = 13
PATH_AUTO, PATH_GEMV, PATH_GEMM, PATH_BAND = 0, 1, 2, 3

# Exported symbols (must match include/shardcompute_hip.h).
EXPORTS = (
    "sc_abi_version",
    "sc_last_error",
    "sc_qmm_bf16",
    "sc_qmm_bf16_path",
    "sc_qmm_bf16_noalloc",
    "sc_qmm_bf16_band",
    "sc_vocab_gather_bf16",
    "sc_qembed_gather_bf16",
    "sc_dequantize_bf16",
    "sc_quantize_affine",
    "sc_qmm_rmsnorm_bf16",
    "sc_qmm_add_rmsnorm_bf16",
    "sc_decode_head_bf16",
    "sc_qmm_swiglu_bf16",
    "sc_rms_norm_bf16",
    "sc_rope_append_kv_bf16",
    "sc_attention_workspace_bytes",
    "sc_attention_bf16",
    "sc_attention_masked_bf16",
    "sc_attention_decode_workspace_bytes",
    "sc_attention_decode_bf16",
    "sc_attention_decode_masked_bf16",
    "sc_silu_mul_bf16",
    "sc_act_bf16",
    "sc_add_row_bias_bf16",
    "sc_argmax_bf16",
    "sc_add_bf16",
    "sc_add_i32",
    "sc_decode_plan_create",
    "sc_decode_plan_run",
    "sc_decode_plan_status",
    "sc_decode_plan_destroy",
    "sc_decode_plan_trace",
    "sc_decode_plan_read_trace",
)

_lib = None
_lock = threading.Lock()

# Optional per-launch timing hook used by the benchmark: when set, every qmm
# launch records a pair of events on the launch stream around the kernel.
timing_sink = None


def load():
    """Open the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m shardcompute_amd.build` "
                "(there is no CPU fallback for the quantized hot path)")
        lib = ctypes.CDLL(LIB_PATH)
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.sc_abi_version.argtypes = []
        lib.sc_abi_version.restype = i32
        lib.sc_last_error.argtypes = []
        lib.sc_last_error.restype = ctypes.c_char_p
        lib.sc_qmm_bf16.argtypes = [p, p, p, p, p, p, i64, i64, i64, i32, i32, p]
        lib.sc_qmm_bf16.restype = i32
        lib.sc_qmm_bf16_path.argtypes = [p, p, p, p, p, p, i64, i64, i64, i32, i32, i32, p]
        lib.sc_qmm_bf16_path.restype = i32
        lib.sc_qmm_bf16_noalloc.argtypes = [p, p, p, p, p, p, i64, i64, i64, i32, i32, p]
        lib.sc_qmm_bf16_noalloc.restype = i32
        lib.sc_qmm_bf16_band.argtypes = [p, p, p, p, p, p, i64, i64, i64, i32, i32, i32, i32, p]
        lib.sc_qmm_bf16_band.restype = i32
        lib.sc_vocab_gather_bf16.argtypes = [p, i32, i64, p, i64, i64, i64, p, p]
        lib.sc_vocab_gather_bf16.restype = i32
        lib.sc_qembed_gather_bf16.argtypes = [p, i32, i64, p, p, p, i64, i64, i64, i32, i32, p, p]
        lib.sc_qembed_gather_bf16.restype = i32
        lib.sc_dequantize_bf16.argtypes = [p, p, p, i64, i64, i32, i32, p, p]
        lib.sc_dequantize_bf16.restype = i32
        lib.sc_quantize_affine.argtypes = [p, i64, i64, i32, i32, p, p, p, p]
        lib.sc_quantize_affine.restype = i32
        f32 = ctypes.c_float
        lib.sc_qmm_rmsnorm_bf16.argtypes = [p, p, p, f32, p, p, p, p, p, p, p, i64, i64, i64, i32, i32, p]
        lib.sc_qmm_rmsnorm_bf16.restype = i32
        lib.sc_qmm_add_rmsnorm_bf16.argtypes = [p, p, p, p, p, p, p, f32, p, p, i64, i64, i64, i32, i32, p]
        lib.sc_qmm_add_rmsnorm_bf16.restype = i32
        lib.sc_decode_head_bf16.argtypes = [p, p, p, f32, p, p, p, p, p, p, p, i64, i64, i64, i32, i32, p, p, i64,
                                            i64, p, p, i64, p, i64, p]
        lib.sc_decode_head_bf16.restype = i32
        lib.sc_qmm_swiglu_bf16.argtypes = [p, p, p, f32, p, p, p, p, p, p, p, p, i64, i64, i64, i32, i32, p]
        lib.sc_qmm_swiglu_bf16.restype = i32
        lib.sc_rms_norm_bf16.argtypes = [p, p, p, p, p, i64, i64, f32, p]
        lib.sc_rms_norm_bf16.restype = i32
        lib.sc_rope_append_kv_bf16.argtypes = [p, i64, i64, i64, i64, i64, i64, p, p, i64, p, p, i64, p, i64, p]
        lib.sc_rope_append_kv_bf16.restype = i32
        lib.sc_attention_workspace_bytes.argtypes = [i64, i64, i64, i64, i64, i64]
        lib.sc_attention_workspace_bytes.restype = i64
        lib.sc_attention_bf16.argtypes = [p, i64, p, p, i64, p, p, i64, i64, i64, i64, i64, i64, f32, p, i64, p]
        lib.sc_attention_bf16.restype = i32
        lib.sc_attention_masked_bf16.argtypes = [p, i64, p, p, i64, p, p, i64, i64, i64, i64, i64, i64, f32, p,
                                                 i64, i64, i64, i64, p, i64, p]
        lib.sc_attention_masked_bf16.restype = i32
        lib.sc_attention_decode_workspace_bytes.argtypes = [i64, i64, i64, i64, i64]
        lib.sc_attention_decode_workspace_bytes.restype = i64
        lib.sc_attention_decode_bf16.argtypes = [p, i64, i64, i64, i64, i64, p, p, i64, p, p, i64, p, i64, f32, p,
                                                 i64, p, i64, p]
        lib.sc_attention_decode_bf16.restype = i32
        lib.sc_attention_decode_masked_bf16.argtypes = [p, i64, i64, i64, i64, i64, p, p, i64, p, p, i64, p, i64, f32,
                                                        p, i64, i64, i64, p, i64, p, i64, p]
        lib.sc_attention_decode_masked_bf16.restype = i32
        lib.sc_silu_mul_bf16.argtypes = [p, i64, i64, p, p]
        lib.sc_silu_mul_bf16.restype = i32
        lib.sc_act_bf16.argtypes = [p, i64, i64, i32, i32, p, p]
        lib.sc_act_bf16.restype = i32
        lib.sc_add_row_bias_bf16.argtypes = [p, i64, i64, p, p, p]
        lib.sc_add_row_bias_bf16.restype = i32
        lib.sc_argmax_bf16.argtypes = [p, i64, i64, p, p, i64, i64, p, p]
        lib.sc_argmax_bf16.restype = i32
        lib.sc_add_bf16.argtypes = [p, p, p, i64, p]
        lib.sc_add_bf16.restype = i32
        lib.sc_add_i32.argtypes = [p, i64, i32, p]
        lib.sc_add_i32.restype = i32
        lib.sc_decode_plan_create.argtypes = [p, p, p]
        lib.sc_decode_plan_create.restype = i32
        lib.sc_decode_plan_run.argtypes = [p, p]
        lib.sc_decode_plan_run.restype = i32
        lib.sc_decode_plan_status.argtypes = [p, p]
        lib.sc_decode_plan_status.restype = i32
        lib.sc_decode_plan_destroy.argtypes = [p]
        lib.sc_decode_plan_destroy.restype = None
        lib.sc_decode_plan_trace.argtypes = [p, i32]
        lib.sc_decode_plan_trace.restype = i32
        lib.sc_decode_plan_read_trace.argtypes = [p, p, i64, p, p]
        lib.sc_decode_plan_read_trace.restype = i32
        v = lib.sc_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libshardcompute_hip ABI {v}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def _check(rc, what):
    if rc != 0:
        msg = load().sc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("shardcompute_amd kernels need GPU tensors (no CPU fallback)")


def _u32(t):
    if t.dtype == torch.uint32:
        return t
    if t.dtype == torch.int32:
        return t.view(torch.uint32)
    raise TypeError(f"packed weights must be uint32 (or int32 bits), got {t.dtype}")


def _bf16(t, name):
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    return t


def qmm(x, wq, scales, biases, bias=None, bits=4, group_size=64, path=PATH_AUTO, out=None, no_alloc=False,
        band_plan=None):
    """y = bf16(x @ dequant(wq, scales, biases)^T) (+ bias), x [..., K] -> [..., N].

    ``no_alloc``: call ``sc_qmm_bf16_noalloc`` (the library allocates nothing;
    pass ``out`` too for a call that allocates nothing at all).
    ``band_plan``: (waves, ksplit) pins the band kernel's plan (``sc_qmm_bf16_band``;
    0 = automatic), for measurements."""
    lib = load()
    _require_gpu(x, wq, scales, biases, bias)
    _bf16(x, "x"), _bf16(scales, "scales"), _bf16(biases, "biases")
    wq = _u32(wq)
    if bias is not None:
        _bf16(bias, "bias")
        bias = bias.contiguous()
    lead = x.shape[:-1]
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    N = wq.shape[0]
    if wq.dim() != 2 or wq.shape[1] * (32 // bits) != K:
        raise ValueError(f"packed weight {tuple(wq.shape)} does not match K={K} at {bits} bits")
    G = K // group_size if group_size else 0
    if scales.shape != (N, G) or biases.shape != (N, G):
        raise ValueError(f"scales/biases must be [{N}, {G}], got {tuple(scales.shape)} / {tuple(biases.shape)}")
    if bias is not None and bias.shape != (N,):
        raise ValueError(f"bias must be [{N}], got {tuple(bias.shape)}")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return y.reshape(*lead, N)
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    sink = timing_sink
    st = _stream(x)
    if sink is not None:
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
    if band_plan is not None:
        if no_alloc or path not in (PATH_AUTO, PATH_BAND):
            raise ValueError("band_plan selects the band kernel (path AUTO or BAND, not no_alloc)")
        rc = lib.sc_qmm_bf16_band(_ptr(x2), _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(y),
                                  M, N, K, bits, group_size, int(band_plan[0]), int(band_plan[1]), st)
    elif no_alloc:
        if path != PATH_AUTO:
            raise ValueError("the allocation-free entry point chooses its kernel itself (path must be AUTO)")
        rc = lib.sc_qmm_bf16_noalloc(_ptr(x2), _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(y),
                                     M, N, K, bits, group_size, st)
    else:
        rc = lib.sc_qmm_bf16_path(_ptr(x2), _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(y),
                                  M, N, K, bits, group_size, path, st)
    if sink is not None:
        ev1.record()
        sink.append((ev0, ev1, M, N, K, bits))
    _check(rc, "sc_qmm_bf16")
    return y.reshape(*lead, N)


def _qmm_common(wq, scales, biases, bias, bits, group_size, K):
    _bf16(scales, "scales"), _bf16(biases, "biases")
    wq = _u32(wq)
    N = wq.shape[0]
    if wq.dim() != 2 or wq.shape[1] * (32 // bits) != K:
        raise ValueError(f"packed weight {tuple(wq.shape)} does not match K={K} at {bits} bits")
    G = K // group_size
    if scales.shape != (N, G) or biases.shape != (N, G):
        raise ValueError(f"scales/biases must be [{N}, {G}], got {tuple(scales.shape)} / {tuple(biases.shape)}")
    if bias is not None:
        _bf16(bias, "bias")
        if bias.shape != (N,):
            raise ValueError(f"bias must be [{N}], got {tuple(bias.shape)}")
        bias = bias.contiguous()
    return wq.contiguous(), scales.contiguous(), biases.contiguous(), bias, N


def _rows(t, K, name):
    if t.dtype != torch.bfloat16 or t.shape[-1] != K or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 [..., {K}] tensor")
    return t


def qmm_rmsnorm(x, norm_weight, eps, wq, scales, biases, residual=None, h_out=None, xn_out=None, bias=None,
                bits=4, group_size=64, out=None):
    """y = qmm(RMSNorm(x + residual)) with the norm fused into the decode GEMV.

    Returns (y, xn); ``h_out`` (when given with a residual) receives x + residual.
    Outputs must be distinct from x and the residual."""
    lib = load()
    _require_gpu(x, norm_weight, wq, scales, biases, residual, h_out, xn_out, bias, out)
    K = x.shape[-1]
    _rows(x, K, "x")
    lead = x.shape[:-1]
    M = x.numel() // K
    wq, scales, biases, bias, N = _qmm_common(wq, scales, biases, bias, bits, group_size, K)
    if residual is not None:
        _rows(residual, K, "residual")
    if h_out is not None:
        _rows(h_out, K, "h_out")
    if norm_weight.shape != (K,) or norm_weight.dtype != torch.bfloat16:
        raise ValueError(f"norm weight must be bf16 [{K}]")
    xn = xn_out if xn_out is not None else torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    _rows(xn, K, "xn_out")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = lib.sc_qmm_rmsnorm_bf16(_ptr(x), _ptr(residual), _ptr(norm_weight.contiguous()), float(eps), _ptr(h_out),
                                 _ptr(xn), _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(y), M, N, K, bits,
                                 group_size, _stream(x))
    _check(rc, "sc_qmm_rmsnorm_bf16")
    return y.reshape(*lead, N), xn.reshape(*lead, K)


def qmm_add_rmsnorm(x, wq, scales, biases, residual, norm_weight, eps, bias=None, bits=4, group_size=64,
                    h_out=None, xn_out=None):
    """y = qmm(x) (+ bias), then h = y + residual and xn = RMSNorm(h): the projection
    before a residual add and the next norm, its split-K pass folded into the norm.
    Returns (h, xn), both [*lead, N]; bit for bit ``qmm`` then ``rms_norm(y,
    residual=residual)``.  Outputs must be distinct from each other and the inputs."""
    lib = load()
    _require_gpu(x, wq, scales, biases, residual, norm_weight, bias, h_out, xn_out)
    K = x.shape[-1]
    _rows(x, K, "x")
    lead = x.shape[:-1]
    M = x.numel() // K
    wq, scales, biases, bias, N = _qmm_common(wq, scales, biases, bias, bits, group_size, K)
    _rows(residual, N, "residual")
    if residual.numel() != M * N:
        raise ValueError(f"residual must hold {M} rows of {N}")
    if norm_weight.shape != (N,) or norm_weight.dtype != torch.bfloat16:
        raise ValueError(f"norm weight must be bf16 [{N}]")
    h = h_out if h_out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    xn = xn_out if xn_out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _rows(h, N, "h_out")
    _rows(xn, N, "xn_out")
    rc = lib.sc_qmm_add_rmsnorm_bf16(_ptr(x), _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(residual),
                                     _ptr(norm_weight.contiguous()), float(eps), _ptr(h), _ptr(xn), M, N, K, bits,
                                     group_size, _stream(x))
    _check(rc, "sc_qmm_add_rmsnorm_bf16")
    return h.reshape(*lead, N), xn.reshape(*lead, N)


DECODE_HEAD_WORKSPACE_BYTES = 16


def decode_head(x, norm_weight, eps, wq, scales, biases, ids, workspace, residual=None, h_out=None, xn_out=None,
                bias=None, bits=4, group_size=64, out=None, tokens=None, step=None, counters=None, n_counters=0):
    """The greedy tail of a decode step: logits = qmm(RMSNorm(x + residual)), then
    ``ids`` (and ``tokens[:, step[0]]``) = the first-max index of each logits row,
    then ``counters[:n_counters] += 1``.  ``workspace``: a zeroed device buffer of
    at least DECODE_HEAD_WORKSPACE_BYTES, left zero by every call.  Returns
    (logits, xn)."""
    lib = load()
    _require_gpu(x, norm_weight, wq, scales, biases, ids, workspace, residual, h_out, xn_out, bias, out, tokens,
                 step, counters)
    K = x.shape[-1]
    _rows(x, K, "x")
    lead = x.shape[:-1]
    M = x.numel() // K
    wq, scales, biases, bias, N = _qmm_common(wq, scales, biases, bias, bits, group_size, K)
    if residual is not None:
        _rows(residual, K, "residual")
    if h_out is not None:
        _rows(h_out, K, "h_out")
    if norm_weight.shape != (K,) or norm_weight.dtype != torch.bfloat16:
        raise ValueError(f"norm weight must be bf16 [{K}]")
    _i32(ids, "ids")
    if ids.numel() != M or not ids.is_contiguous():
        raise ValueError(f"ids must be a contiguous int32 buffer of {M} entries")
    if workspace.nbytes < DECODE_HEAD_WORKSPACE_BYTES or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous buffer of at least {DECODE_HEAD_WORKSPACE_BYTES} bytes")
    if tokens is not None:
        _i32(tokens, "tokens")
        if tokens.dim() != 2 or tokens.shape[0] != M or tokens.stride(1) != 1:
            raise ValueError("tokens must be a row-major [rows, n] int32 matrix")
    if n_counters:
        _i32(counters, "counters")
        if counters.numel() < n_counters or not counters.is_contiguous():
            raise ValueError(f"counters must hold {n_counters} contiguous int32 entries")
    xn = xn_out if xn_out is not None else torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    _rows(xn, K, "xn_out")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    rc = lib.sc_decode_head_bf16(_ptr(x), _ptr(residual), _ptr(norm_weight.contiguous()), float(eps), _ptr(h_out),
                                 _ptr(xn), _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(y), M, N, K, bits,
                                 group_size, _ptr(ids), _ptr(tokens), tokens.stride(0) if tokens is not None else 0,
                                 tokens.shape[1] if tokens is not None else 0, _ptr(step),
                                 _ptr(counters) if n_counters else None, int(n_counters), _ptr(workspace),
                                 workspace.nbytes, _stream(x))
    _check(rc, "sc_decode_head_bf16")
    return y.reshape(*lead, N), xn.reshape(*lead, K)


def qmm_swiglu(x, wq, scales, biases, norm_weight=None, eps=1e-5, residual=None, h_out=None, xn_out=None,
               bias=None, bits=4, group_size=64, act_out=None, gate_up_scratch=None):
    """act = silu(gate) * up for the stacked gate|up weight [2I, ...] applied to x,
    or to RMSNorm(x + residual) when ``norm_weight`` is given.  Returns (act, xn)."""
    lib = load()
    _require_gpu(x, wq, scales, biases, norm_weight, residual, h_out, xn_out, bias, act_out, gate_up_scratch)
    K = x.shape[-1]
    _rows(x, K, "x")
    lead = x.shape[:-1]
    M = x.numel() // K
    wq, scales, biases, bias, N = _qmm_common(wq, scales, biases, bias, bits, group_size, K)
    if N % 16:
        raise ValueError(f"gate|up rows ({N}) must be 2 * I with I a multiple of 8")
    I = N // 2
    xn = None
    if norm_weight is not None:
        if norm_weight.shape != (K,) or norm_weight.dtype != torch.bfloat16:
            raise ValueError(f"norm weight must be bf16 [{K}]")
        xn = xn_out if xn_out is not None else torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
        _rows(xn, K, "xn_out")
        norm_weight = norm_weight.contiguous()
    elif residual is not None:
        raise ValueError("a residual needs the norm weight")
    if residual is not None:
        _rows(residual, K, "residual")
    act = act_out if act_out is not None else torch.empty((M, I), dtype=torch.bfloat16, device=x.device)
    _rows(act, I, "act_out")
    gu = gate_up_scratch if gate_up_scratch is not None else torch.empty((M, N), dtype=torch.bfloat16,
                                                                          device=x.device)
    _rows(gu, N, "gate_up_scratch")
    rc = lib.sc_qmm_swiglu_bf16(_ptr(x), _ptr(residual), _ptr(norm_weight), float(eps), _ptr(h_out), _ptr(xn),
                                _ptr(wq), _ptr(scales), _ptr(biases), _ptr(bias), _ptr(act), _ptr(gu), M, I, K, bits,
                                group_size, _stream(x))
    _check(rc, "sc_qmm_swiglu_bf16")
    return act.reshape(*lead, I), (xn.reshape(*lead, K) if xn is not None else None)


def vocab_gather(ids, table, vocab_start=0, out=None):
    """Masked bf16 row gather: ids [...] -> [..., D]; out-of-shard ids give +0 rows."""
    lib = load()
    _require_gpu(ids, table)
    _bf16(table, "table")
    if ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"ids must be int32 or int64, got {ids.dtype}")
    table = table.contiguous()
    idc = ids.contiguous()
    V, D = table.shape
    res = out if out is not None else torch.empty(tuple(ids.shape) + (D,), dtype=torch.bfloat16,
                                                  device=table.device)
    rc = lib.sc_vocab_gather_bf16(_ptr(idc), 1 if idc.dtype == torch.int64 else 0, idc.numel(), _ptr(table),
                                  V, D, int(vocab_start), _ptr(res), _stream(table))
    _check(rc, "sc_vocab_gather_bf16")
    return res


def qembed_gather(ids, wq, scales, biases, vocab_start=0, bits=4, group_size=64):
    """Masked gather + dequantize of a quantized table: ids [...] -> bf16 [..., D]."""
    lib = load()
    _require_gpu(ids, wq, scales, biases)
    wq = _u32(wq).contiguous()
    _bf16(scales, "scales"), _bf16(biases, "biases")
    if ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"ids must be int32 or int64, got {ids.dtype}")
    V = wq.shape[0]
    D = wq.shape[1] * (32 // bits)
    idc = ids.contiguous()
    res = torch.empty(tuple(ids.shape) + (D,), dtype=torch.bfloat16, device=wq.device)
    rc = lib.sc_qembed_gather_bf16(_ptr(idc), 1 if idc.dtype == torch.int64 else 0, idc.numel(), _ptr(wq),
                                   _ptr(scales.contiguous()), _ptr(biases.contiguous()), V, D, int(vocab_start),
                                   bits, group_size, _ptr(res), _stream(wq))
    _check(rc, "sc_qembed_gather_bf16")
    return res


def dequantize(wq, scales, biases, bits=4, group_size=64):
    """bf16(scales * q + biases) for a whole packed matrix -> [rows, K]."""
    lib = load()
    _require_gpu(wq, scales, biases)
    wq = _u32(wq).contiguous()
    rows = wq.shape[0]
    K = wq.shape[1] * (32 // bits)
    out = torch.empty((rows, K), dtype=torch.bfloat16, device=wq.device)
    rc = lib.sc_dequantize_bf16(_ptr(wq), _ptr(_bf16(scales, "scales").contiguous()),
                                _ptr(_bf16(biases, "biases").contiguous()), rows, K, bits, group_size, _ptr(out),
                                _stream(wq))
    _check(rc, "sc_dequantize_bf16")
    return out


def quantize(w, bits=4, group_size=64):
    """MLX affine quantizer on the GPU: fp32 [rows, K] -> (uint32 wq, bf16 scales, bf16 biases)."""
    lib = load()
    _require_gpu(w)
    if w.dim() != 2:
        raise ValueError("quantize expects a 2-D weight")
    w = w.to(torch.float32).contiguous()
    rows, K = w.shape
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if K % group_size:
        raise ValueError(f"K={K} must be a multiple of group_size={group_size}")
    wq = torch.empty((rows, K * bits // 32), dtype=torch.uint32, device=w.device)
    s = torch.empty((rows, K // group_size), dtype=torch.bfloat16, device=w.device)
    b = torch.empty_like(s)
    rc = lib.sc_quantize_affine(_ptr(w), rows, K, bits, group_size, _ptr(wq), _ptr(s), _ptr(b), _stream(w))
    _check(rc, "sc_quantize_affine")
    return wq, s, b


# ---------------------------------------------------------------- decoder wiring


def _i32(t, name):
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    return t


def rms_norm(x, weight, eps, residual=None, h_out=None, out=None):
    """y = (h / sqrt(mean(h*h) + eps)) * weight with h = x (+ residual, stored in h_out).

    x, residual [..., D] bf16; weight [D] bf16.  Returns y (same shape as x).
    """
    lib = load()
    _require_gpu(x, weight, residual, h_out, out)
    _bf16(x, "x"), _bf16(weight, "weight")
    D = x.shape[-1]
    if weight.shape != (D,):
        raise ValueError(f"weight must be [{D}], got {tuple(weight.shape)}")
    if not x.is_contiguous():
        x = x.contiguous()
    if residual is not None:
        _bf16(residual, "residual")
        if residual.shape != x.shape or not residual.is_contiguous():
            raise ValueError("residual must be a contiguous tensor of x's shape")
    for t in (h_out, out):
        if t is not None and (t.shape != x.shape or t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError("h_out/out must be contiguous bf16 tensors of x's shape")
    y = out if out is not None else torch.empty_like(x)
    rows = x.numel() // D if D else 0
    rc = lib.sc_rms_norm_bf16(_ptr(x), _ptr(residual), _ptr(weight.contiguous()), _ptr(y), _ptr(h_out), rows, D,
                              float(eps), _stream(x))
    _check(rc, "sc_rms_norm_bf16")
    return y


def rope_append_kv(qkv, B, S, H, Hkv, D, cos_t, sin_t, k_cache, v_cache_t, cache_len, pos_offset=0):
    """RoPE on the q/k heads of the fused rows qkv [B*S, >= (H+2Hkv)*D] (q in place)
    and append of k, v at cache slots cache_len[0] + s (rotary position + pos_offset).

    The caller guarantees room: cache_len[0] + S <= capacity and the tables cover
    every rotary position (the kernel skips tokens that would fall outside)."""
    lib = load()
    _require_gpu(qkv, cos_t, sin_t, k_cache, v_cache_t, cache_len)
    _bf16(qkv, "qkv"), _bf16(k_cache, "k_cache"), _bf16(v_cache_t, "v_cache_t"), _i32(cache_len, "cache_len")
    if qkv.dim() != 2 or qkv.shape[0] != B * S or qkv.stride(1) != 1:
        raise ValueError(f"qkv must be a row-major [{B * S}, *] matrix")
    T_cap = k_cache.shape[2]
    if tuple(k_cache.shape) != (B, Hkv, T_cap, D) or tuple(v_cache_t.shape) != (B, Hkv, D, T_cap):
        raise ValueError("cache shapes must be K [B, Hkv, T_cap, D] and Vt [B, Hkv, D, T_cap]")
    if not (k_cache.is_contiguous() and v_cache_t.is_contiguous()):
        raise ValueError("cache tensors must be contiguous")
    if (cos_t.dtype != torch.float32 or sin_t.dtype != torch.float32 or cos_t.shape != sin_t.shape
            or cos_t.dim() != 2 or cos_t.shape[1] != D // 2 or not cos_t.is_contiguous() or not sin_t.is_contiguous()):
        raise ValueError("cos/sin tables must be contiguous fp32 [L, D/2]")
    rc = lib.sc_rope_append_kv_bf16(_ptr(qkv), qkv.stride(0), B, S, H, Hkv, D, _ptr(cos_t), _ptr(sin_t),
                                    cos_t.shape[0], _ptr(k_cache), _ptr(v_cache_t), T_cap, _ptr(cache_len),
                                    int(pos_offset), _stream(qkv))
    _check(rc, "sc_rope_append_kv_bf16")


def attention_workspace_bytes(B, S, H, Hkv, D, T_cap):
    return int(load().sc_attention_workspace_bytes(B, S, H, Hkv, D, T_cap))


def attention(q, B, S, H, Hkv, D, k_cache, v_cache_t, cache_len, scale, out=None, workspace=None, mask=None,
              n_keys=None):
    """Causal GQA attention of the S new positions (rows of q [B*S, >= H*D]) against
    the cache: cache_len[0] earlier positions followed by the S new ones.
    Returns out [B*S, H*D] bf16.

    ``mask``: an additive mask broadcastable to ``[B, H, S, n_keys]`` (``n_keys`` =
    cache_len[0] + S, which the caller states: the length is a device counter),
    added to the scaled scores before the causal mask (``attention.py:449-450``)."""
    lib = load()
    _require_gpu(q, k_cache, v_cache_t, cache_len, out, workspace, mask)
    _bf16(q, "q"), _i32(cache_len, "cache_len")
    if q.dim() != 2 or q.shape[0] != B * S or q.stride(1) != 1:
        raise ValueError(f"q must be a row-major [{B * S}, *] matrix")
    T_cap = k_cache.shape[2]
    if out is None:
        out = torch.empty((B * S, H * D), dtype=torch.bfloat16, device=q.device)
    need = attention_workspace_bytes(B, S, H, Hkv, D, T_cap)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if mask is None:
        rc = lib.sc_attention_bf16(_ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache_t), T_cap, _ptr(cache_len),
                                   _ptr(out), out.stride(0), B, S, H, Hkv, D, float(scale), _ptr(workspace),
                                   ws_bytes, _stream(q))
        _check(rc, "sc_attention_bf16")
        return out
    m = broadcast_mask(mask, B, H, S, n_keys)
    rc = lib.sc_attention_masked_bf16(_ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache_t), T_cap, _ptr(cache_len),
                                      _ptr(out), out.stride(0), B, S, H, Hkv, D, float(scale), _ptr(m), *m.stride(),
                                      _ptr(workspace), ws_bytes, _stream(q))
    _check(rc, "sc_attention_masked_bf16")
    return out


def broadcast_mask(mask, B, H, S, n_keys):
    """An additive attention mask as an fp32 view of shape ``[B, H, S, n_keys]`` whose
    broadcast dimensions have stride 0 (the layout sc_attention_masked_bf16 reads).
    Raises ValueError when the mask does not broadcast to that shape."""
    if n_keys is None:
        raise ValueError("a masked attention call needs n_keys (cache length + S)")
    if not isinstance(mask, torch.Tensor):
        raise TypeError("attention mask must be a torch tensor on the GPU")
    m = mask if mask.dtype == torch.float32 else mask.float()
    if m.dim() > 4:
        raise ValueError(f"attention mask has {m.dim()} dimensions (at most 4)")
    while m.dim() < 4:
        m = m.unsqueeze(0)
    try:
        return torch.broadcast_to(m, (B, H, S, n_keys))
    except RuntimeError as e:
        raise ValueError(f"attention mask of shape {tuple(mask.shape)} does not broadcast to "
                         f"[{B}, {H}, {S}, {n_keys}]") from e


def attention_decode_workspace_bytes(B, H, Hkv, D, T_cap):
    return int(load().sc_attention_decode_workspace_bytes(B, H, Hkv, D, T_cap))


def attention_decode(qkv, B, H, Hkv, D, cos_t, sin_t, k_cache, v_cache_t, cache_len, scale, pos_offset=0, out=None,
                     workspace=None, mask=None, n_keys=None):
    """One decode step of attention: RoPE of row b's q and k heads (rotary position
    cache_len[0] + pos_offset), append of k and v at slot cache_len[0], and
    attention of the new position over the cache.  qkv [B, >= (H + 2Hkv) * D] is
    not modified.  ``mask``: the reference's additive attention mask, broadcastable
    to [B, H, 1, n_keys] (n_keys = cached positions + 1).  Returns out [B, H*D] bf16."""
    lib = load()
    _require_gpu(qkv, cos_t, sin_t, k_cache, v_cache_t, cache_len, out, workspace)
    _bf16(qkv, "qkv"), _bf16(k_cache, "k_cache"), _bf16(v_cache_t, "v_cache_t"), _i32(cache_len, "cache_len")
    if qkv.dim() != 2 or qkv.shape[0] != B or qkv.stride(1) != 1:
        raise ValueError(f"qkv must be a row-major [{B}, *] matrix")
    T_cap = k_cache.shape[2]
    if tuple(k_cache.shape) != (B, Hkv, T_cap, D) or tuple(v_cache_t.shape) != (B, Hkv, D, T_cap):
        raise ValueError("cache shapes must be k [B, Hkv, T_cap, D] and v^T [B, Hkv, D, T_cap]")
    if (cos_t.dtype != torch.float32 or sin_t.dtype != torch.float32 or cos_t.shape != sin_t.shape
            or cos_t.dim() != 2 or cos_t.shape[1] != D // 2 or not cos_t.is_contiguous() or not sin_t.is_contiguous()):
        raise ValueError("cos/sin tables must be contiguous fp32 [L, D/2]")
    if out is None:
        out = torch.empty((B, H * D), dtype=torch.bfloat16, device=qkv.device)
    need = attention_decode_workspace_bytes(B, H, Hkv, D, T_cap)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=qkv.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if mask is not None:
        m = broadcast_mask(mask, B, H, 1, n_keys)
        sb, sh, _, st = m.stride()
        rc = lib.sc_attention_decode_masked_bf16(_ptr(qkv), qkv.stride(0), B, H, Hkv, D, _ptr(cos_t), _ptr(sin_t),
                                                 cos_t.shape[0], _ptr(k_cache), _ptr(v_cache_t), T_cap,
                                                 _ptr(cache_len), int(pos_offset), float(scale), _ptr(m), sb, sh, st,
                                                 _ptr(out), out.stride(0), _ptr(workspace), ws_bytes, _stream(qkv))
        _check(rc, "sc_attention_decode_masked_bf16")
        return out
    rc = lib.sc_attention_decode_bf16(_ptr(qkv), qkv.stride(0), B, H, Hkv, D, _ptr(cos_t), _ptr(sin_t),
                                      cos_t.shape[0], _ptr(k_cache), _ptr(v_cache_t), T_cap, _ptr(cache_len),
                                      int(pos_offset), float(scale), _ptr(out), out.stride(0), _ptr(workspace),
                                      ws_bytes, _stream(qkv))
    _check(rc, "sc_attention_decode_bf16")
    return out


def silu_mul(gate_up, out=None):
    """silu(gate) * up for gate_up [..., 2I] (gate first) -> [..., I] bf16."""
    lib = load()
    _require_gpu(gate_up, out)
    _bf16(gate_up, "gate_up")
    gate_up = gate_up.contiguous()
    I2 = gate_up.shape[-1]
    if I2 % 2:
        raise ValueError("gate_up width must be even")
    I = I2 // 2
    rows = gate_up.numel() // I2 if I2 else 0
    if out is None:
        out = torch.empty(gate_up.shape[:-1] + (I,), dtype=torch.bfloat16, device=gate_up.device)
    rc = lib.sc_silu_mul_bf16(_ptr(gate_up), rows, I, _ptr(out), _stream(gate_up))
    _check(rc, "sc_silu_mul_bf16")
    return out


ACT_KINDS = {"silu": 0, "swish": 0, "gelu": 1, "gelu_new": 2, "relu": 3, "gelu_exact": 4}


def act(x, activation, gated, out=None):
    """The MLP activation by name (``ParallelMLP``'s names): gated, f(gate) * up for
    x = gate|up [..., 2I] -> [..., I]; ungated, f(x) for x [..., I] -> [..., I]."""
    lib = load()
    _require_gpu(x, out)
    _bf16(x, "x")
    if activation not in ACT_KINDS:
        raise ValueError(f"Unknown activation: {activation}")
    x = x.contiguous()
    W = x.shape[-1]
    if gated and W % 2:
        raise ValueError("gate_up width must be even")
    I = W // 2 if gated else W
    rows = x.numel() // W if W else 0
    if out is None:
        out = torch.empty(x.shape[:-1] + (I,), dtype=torch.bfloat16, device=x.device)
    rc = lib.sc_act_bf16(_ptr(x), rows, I, ACT_KINDS[activation], 1 if gated else 0, _ptr(out), _stream(x))
    _check(rc, "sc_act_bf16")
    return out


def add_row_bias(x, bias, out=None):
    """x [..., D] + bias [D] per row, rounded to bf16 (out may be x)."""
    lib = load()
    _require_gpu(x, bias, out)
    _bf16(x, "x"), _bf16(bias, "bias")
    x = x.contiguous()
    D = x.shape[-1]
    if tuple(bias.shape) != (D,):
        raise ValueError(f"bias must be [{D}], got {tuple(bias.shape)}")
    if out is None:
        out = torch.empty_like(x)
    rows = x.numel() // D if D else 0
    rc = lib.sc_add_row_bias_bf16(_ptr(x), rows, D, _ptr(bias.contiguous()), _ptr(out), _stream(x))
    _check(rc, "sc_add_row_bias_bf16")
    return out


def argmax(logits, ids=None, tokens=None, step=None):
    """First-max index of each row of logits [rows, V] bf16 -> int32 [rows].

    With ``tokens`` ([rows, n] int32) the ids are also stored at column step[0]."""
    lib = load()
    _require_gpu(logits, ids, tokens, step)
    _bf16(logits, "logits")
    logits = logits.reshape(-1, logits.shape[-1]).contiguous()
    rows, V = logits.shape
    if ids is None:
        ids = torch.empty(rows, dtype=torch.int32, device=logits.device)
    _i32(ids, "ids")
    if tokens is not None:
        _i32(tokens, "tokens")
        if tokens.dim() != 2 or tokens.shape[0] != rows or tokens.stride(1) != 1:
            raise ValueError("tokens must be a row-major [rows, n] int32 matrix")
    rc = lib.sc_argmax_bf16(_ptr(logits), rows, V, _ptr(ids), _ptr(tokens),
                            tokens.stride(0) if tokens is not None else 0,
                            tokens.shape[1] if tokens is not None else 0, _ptr(step), _stream(logits))
    _check(rc, "sc_argmax_bf16")
    return ids


def add(a, b, out=None):
    """bf16(a + b) elementwise for same-shape bf16 tensors."""
    lib = load()
    _require_gpu(a, b, out)
    _bf16(a, "a"), _bf16(b, "b")
    if a.shape != b.shape:
        raise ValueError(f"shapes differ: {tuple(a.shape)} vs {tuple(b.shape)}")
    a, b = a.contiguous(), b.contiguous()
    out = torch.empty_like(a) if out is None else out
    rc = lib.sc_add_bf16(_ptr(a), _ptr(b), _ptr(out), a.numel(), _stream(a))
    _check(rc, "sc_add_bf16")
    return out


def add_i32(counters, delta, n=None):
    """counters[:n] += delta on the stream (device-side step bookkeeping)."""
    lib = load()
    _require_gpu(counters)
    _i32(counters, "counters")
    n = counters.numel() if n is None else n
    rc = lib.sc_add_i32(_ptr(counters), n, int(delta), _stream(counters))
    _check(rc, "sc_add_i32")
