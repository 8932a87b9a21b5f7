"""CPU oracle for the quantized-inference hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path the
HIP library replaces:

* ``mlx_affine``  — MLX's affine 4/8-bit group quantization format
  (``mx.quantize`` / ``mx.dequantize`` / ``mx.quantized_matmul(transpose=True)``)
  as called from ``src/shardcompute/parallel/quantized_linear.py:116-120,168-176``
  and ``src/shardcompute/model/quantization.py:44-75,117``.
* ``gather``      — the vocab-sharded masked row gather of
  ``src/shardcompute/parallel/embedding.py:322-356`` (offset, range mask, clip,
  take, zero out-of-shard rows), on a bf16 table and on a quantized table.
* ``decoder``     — the layer wiring of ``parallel/attention.py``,
  ``parallel/mlp.py``, ``parallel/transformer.py`` and the greedy loop of
  ``worker/executor.py:229-347``, in numpy.
* ``cref``        — ctypes binding of ``qmm_ref.c``, an OpenMP C restatement of
  the same quantized matmul / gather, used as a second independent
  implementation and as the timed CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import anything from here, and only to check results against (or, for
the baseline, to time the CPU), never as the thing measured.  The product path
(``shardcompute_amd``) never imports it: it fails loudly when the HIP library
is missing instead of falling back to the CPU.

Parity status (what pins each function) is listed per function in the module
docstrings.  Functions that nothing external pins carry the words
"parity unpinned" there.
"""
