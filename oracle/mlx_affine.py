"""MLX affine group quantization, restated in numpy — TEST INFRASTRUCTURE ONLY.

The reference never implements the arithmetic itself: it calls the third-party
package ``mlx`` (pinned only as ``mlx>=0.12.0``, ``requirements.txt:2``,
``pyproject.toml:37``; not vendored, not importable in this image).  Call sites:

* ``mx.quantize(w_f32, group_size, bits)``  ``parallel/quantized_linear.py:116-120``,
  ``:353-357``, ``parallel/embedding.py:303-307``, ``model/quantization.py:117,148``
* ``mx.dequantize(wq, s, b, group_size, bits)``  ``parallel/embedding.py:343-349,373-379``,
  ``model/quantization.py:44-52``
* ``mx.quantized_matmul(x, wq, s, b, transpose=True, group_size, bits)``
  ``parallel/quantized_linear.py:168-176,206-214,435-443,472-480``,
  ``parallel/transformer.py:639-647,971-979``, ``model/quantization.py:67-75``

Format (MLX's published convention; the in-repo statements are
``parallel/embedding.py:202-205`` "8 values per uint32" with scales/biases
``[rows, D / group_size]`` and ``parallel/quantized_linear.py:393``
``pack_factor = 32 // bits``):

* a row of K values is cut into groups of ``group_size`` consecutive values;
  each group has one scale ``s`` and one bias ``b``; ``w ~= s * q + b`` with
  ``q`` an unsigned ``bits``-bit integer;
* ``32 // bits`` consecutive values of a row share one uint32 word, value ``j``
  of the word in bits ``[j*bits, (j+1)*bits)`` (least significant first).

Parity status
-------------
* ``pack`` / ``unpack``: LSB-first element order is MLX's convention; no file of
  the reference pins it (parity unpinned against MLX).  Pinned internally by a
  hand-written known-answer word and by an independent bit-string unpacker.
* ``dequantize`` / ``quantized_matmul``: the formula ``s*q + b`` and the
  ``transpose=True`` contraction ``y = x @ W^T`` are pinned by closed forms
  (one-hot q, s = 0, constant groups), by an independent per-element loop, and
  by the reference tests' shard invariants (column concat == full, row partial
  sum == full).  MLX's own accumulation precision for bf16 inputs is not
  pinned (parity unpinned); this oracle accumulates in float64, i.e. it gives
  the exact value of the affine formula on the given bf16 inputs.
* ``quantize``: the edge-preserving rule of current MLX releases.  Its exact
  output is MLX-version dependent and pinned only by properties (range, error
  bound of half a step, exact edge, monotone codes); it is fixture plumbing,
  since both sides of every comparison receive the same packed weights.
"""
import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16

SUPPORTED_BITS = (4, 8)


def _check(bits, group_size):
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if group_size <= 0 or group_size % (32 // bits) != 0:
        raise ValueError(f"group_size {group_size} incompatible with bits {bits}")


def pack(q, bits):
    """uint codes [R, K] -> uint32 words [R, K * bits / 32], LSB first."""
    q = np.asarray(q, dtype=np.uint32)
    pf = 32 // bits
    R, K = q.shape
    if K % pf:
        raise ValueError("K must be a multiple of 32 / bits")
    q = q.reshape(R, K // pf, pf)
    shifts = (np.arange(pf, dtype=np.uint32) * np.uint32(bits))
    return np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)


def unpack(wq, bits):
    """uint32 words [R, W] -> uint codes [R, W * 32 / bits] (uint8)."""
    wq = np.asarray(wq, dtype=np.uint32)
    pf = 32 // bits
    mask = np.uint32((1 << bits) - 1)
    shifts = (np.arange(pf, dtype=np.uint32) * np.uint32(bits))
    q = (wq[..., None] >> shifts) & mask
    return q.reshape(wq.shape[0], -1).astype(np.uint8)


def quantize(w, group_size=64, bits=4):
    """float32 [R, K] -> (wq uint32, scales f32 [R, G], biases f32 [R, G]).

    Per group (MLX's affine quantizer, edge-preserving variant):
    ``scale = max((wmax - wmin) / n_bins, 1e-7)``; the edge is the end with the
    larger magnitude (``wmin`` if ``|wmin| > |wmax|``, else ``wmax`` with a
    negated scale); ``q0 = round(edge / scale)``; if ``q0 != 0`` the scale is
    refit to ``edge / q0`` and the bias is the edge, else the bias is 0;
    ``q = clip(round((w - bias) / scale), 0, n_bins)``.  All in float32,
    ``round`` is round-half-to-even.
    """
    _check(bits, group_size)
    w = np.asarray(w, dtype=np.float32)
    R, K = w.shape
    if K % group_size:
        raise ValueError(f"K={K} must be a multiple of group_size={group_size}")
    n_bins = np.float32((1 << bits) - 1)
    g = w.reshape(R, K // group_size, group_size)
    wmax = g.max(axis=-1)
    wmin = g.min(axis=-1)
    scale = np.maximum((wmax - wmin) / n_bins, np.float32(1e-7)).astype(np.float32)
    use_min = np.abs(wmin) > np.abs(wmax)
    scale = np.where(use_min, scale, -scale).astype(np.float32)
    edge = np.where(use_min, wmin, wmax).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    nz = q0 != 0
    safe_q0 = np.where(nz, q0, np.float32(1))
    scale = np.where(nz, edge / safe_q0, scale).astype(np.float32)
    bias = np.where(nz, edge, np.float32(0)).astype(np.float32)
    q = np.rint((g - bias[..., None]) / scale[..., None])
    q = np.clip(q, 0, n_bins).astype(np.uint32).reshape(R, K)
    return pack(q, bits), scale, bias


def quantize_bf16(w, group_size=64, bits=4):
    """``quantize`` then round scales and biases to bf16 (uint16 patterns)."""
    wq, s, b = quantize(w, group_size, bits)
    return wq, f32_to_bf16(s), f32_to_bf16(b)


def dequantize_f64(wq, scales, biases, group_size=64, bits=4):
    """Exact dequantized weights ``s*q + b`` in float64, shape [R, K].

    ``scales`` / ``biases`` are uint16 bf16 patterns or float arrays.
    """
    _check(bits, group_size)
    q = unpack(wq, bits).astype(np.float64)
    s = _as_f64(scales)
    b = _as_f64(biases)
    R, K = q.shape
    G = K // group_size
    if s.shape != (R, G) or b.shape != (R, G):
        raise ValueError(f"scales/biases must be [{R}, {G}], got {s.shape} / {b.shape}")
    qg = q.reshape(R, G, group_size)
    return (s[..., None] * qg + b[..., None]).reshape(R, K)


def dequantize_bf16(wq, scales, biases, group_size=64, bits=4):
    """``mx.dequantize`` with bf16 scales/biases -> uint16 bf16 [R, K].

    Each value is ``bf16(float32(s * q) + b)``: the product is exact in fp32,
    the add rounds once to fp32, then once to bf16 (RNE).  This is the
    definition the HIP dequant-gather is required to match bit for bit.
    MLX's own rounding for this op is not pinned (parity unpinned).
    """
    _check(bits, group_size)
    q = unpack(wq, bits).astype(np.float32)
    s = bf16_to_f32(scales)
    b = bf16_to_f32(biases)
    R, K = q.shape
    G = K // group_size
    qg = q.reshape(R, G, group_size)
    v = (s[..., None] * qg).astype(np.float32) + b[..., None]
    return f32_to_bf16(v.astype(np.float32).reshape(R, K))


def quantized_matmul_f64(x, wq, scales, biases, group_size=64, bits=4, row_block=2048):
    """``mx.quantized_matmul(x, wq, s, b, transpose=True)`` in float64.

    ``x``: uint16 bf16 [M, K] (or float array); returns float64 [M, N] with
    ``y[m, n] = sum_k x[m, k] * (s[n, k // gs] * q[n, k] + b[n, k // gs])``.
    """
    xf = _as_f64(x)
    wq = np.asarray(wq, dtype=np.uint32)
    N = wq.shape[0]
    K = wq.shape[1] * (32 // bits)
    if xf.shape[-1] != K:
        raise ValueError(f"x last dim {xf.shape[-1]} != K {K}")
    out = np.empty((xf.shape[0], N), dtype=np.float64)
    for r0 in range(0, N, row_block):
        r1 = min(N, r0 + row_block)
        w = dequantize_f64(wq[r0:r1], np.asarray(scales)[r0:r1], np.asarray(biases)[r0:r1],
                           group_size, bits)
        out[:, r0:r1] = xf @ w.T
    return out


def quantized_matmul_bf16(x, wq, scales, biases, bias=None, group_size=64, bits=4):
    """Quantized linear as the reference layer computes it -> uint16 bf16 [M, N].

    ``output = bf16(qmm(x))`` then, if a linear bias is present,
    ``output = bf16(output + bias)`` (``parallel/quantized_linear.py:168-180``:
    the bf16 result of ``mx.quantized_matmul`` plus the bf16 bias).
    """
    y = f32_to_bf16(quantized_matmul_f64(x, wq, scales, biases, group_size, bits).astype(np.float32))
    if bias is not None:
        y = f32_to_bf16(bf16_to_f32(y) + bf16_to_f32(np.asarray(bias))[None, :])
    return y


def _as_f64(a):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return bf16_to_f32(a).astype(np.float64)
    return a.astype(np.float64)
