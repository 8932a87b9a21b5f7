"""Writes the golden fixtures of the quantized path (run: python tests/golden/make_golden.py).

The reference holds no golden vectors for this path and MLX is not importable,
so the expected outputs come from the oracle (``oracle/``), which the CPU
tests pin by closed forms, independent implementations and invariants.  The
fixtures freeze those outputs on small seeded inputs so that the GPU tests and
any later change of the oracle are checked against the same bytes.

Every file is a plain ``.npz`` of arrays (no pickles): bf16 values are uint16
bit patterns, packed weights uint32.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.bf16 import f32_to_bf16  # noqa: E402
from oracle.gather import qembed_gather_bf16, vocab_gather_bf16  # noqa: E402
from oracle.mlx_affine import quantize_bf16, quantized_matmul_bf16  # noqa: E402

QMM_CASES = [  # (M, K, N, bits, with_bias)
    (1, 128, 64, 4, False), (1, 512, 96, 8, True), (3, 256, 96, 4, True), (8, 512, 40, 4, False),
    (8, 320, 72, 8, False), (32, 256, 130, 4, True), (32, 192, 64, 8, True), (130, 192, 64, 4, False),
    (130, 256, 136, 8, True), (17, 1024, 33, 4, True),
]


def make_qmm(rng):
    out = {}
    for i, (M, K, N, bits, with_bias) in enumerate(QMM_CASES):
        x = f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        wq, s, b = quantize_bf16(w, 64, bits)
        bias = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1) if with_bias else None
        y = quantized_matmul_bf16(x, wq, s, b, bias, 64, bits)
        p = f"c{i}_"
        out.update({p + "x": x, p + "wq": wq, p + "s": s, p + "b": b, p + "y": y,
                    p + "meta": np.array([M, K, N, bits, int(with_bias)], np.int64)})
        if bias is not None:
            out[p + "bias"] = bias
    out["n_cases"] = np.array(len(QMM_CASES))
    return out


def make_gather(rng):
    V, D, start = 50, 24, 100
    table = f32_to_bf16(rng.standard_normal((V, D)).astype(np.float32) * 0.02)
    table[1, :4] = [0x8000, 0x7FC1, 0x7F80, 0xFF80]  # -0.0, NaN payload, +Inf, -Inf
    table[2, :] = 0x8000
    ids = np.array([start - 1, start, start + 1, start + 2, start + V - 1, start + V, -1, -5000, 0, 10 ** 6,
                    start + 17, start + 17], np.int64).reshape(2, 6)
    vt = f32_to_bf16(rng.standard_normal((64, 136)).astype(np.float32))  # D % 8 == 0, vector path
    vids = rng.integers(-20, 200, size=(5, 7)).astype(np.int32)
    odd = f32_to_bf16(rng.standard_normal((30, 13)).astype(np.float32))  # D % 8 != 0, scalar path
    oids = rng.integers(0, 60, size=(9,)).astype(np.int64)
    return {"table": table, "ids": ids, "start": np.array(start), "out": vocab_gather_bf16(ids, table, start),
            "vtable": vt, "vids": vids, "vstart": np.array(64), "vout": vocab_gather_bf16(vids, vt, 64),
            "otable": odd, "oids": oids, "ostart": np.array(30), "oout": vocab_gather_bf16(oids, odd, 30)}


def make_qembed(rng):
    out = {}
    for bits in (4, 8):
        V, D, start = 40, 192, 40
        w = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
        wq, s, b = quantize_bf16(w, 64, bits)
        ids = np.array([[39, 40, 41, 79], [80, 55, -1, 60]], np.int64)
        out.update({f"w{bits}_wq": wq, f"w{bits}_s": s, f"w{bits}_b": b, f"w{bits}_ids": ids,
                    f"w{bits}_out": qembed_gather_bf16(ids, wq, s, b, start, 64, bits)})
    out["start"] = np.array(40)
    return out


def make_quantize(rng):
    w = (rng.standard_normal((24, 320)) * 0.02).astype(np.float32)
    w[0, :64] = 0.37
    w[1, :64] = 0.0
    w[2, 64:128] = -1.5
    w[3, :] = np.linspace(-1, 1, 320, dtype=np.float32)
    out = {"w": w}
    for bits in (4, 8):
        wq, s, b = quantize_bf16(w, 64, bits)
        out.update({f"wq{bits}": wq, f"s{bits}": s, f"b{bits}": b})
    return out


def main():
    rng = np.random.default_rng(20260101)
    np.savez_compressed(os.path.join(HERE, "qmm_cases.npz"), **make_qmm(rng))
    np.savez_compressed(os.path.join(HERE, "gather_cases.npz"), **make_gather(rng))
    np.savez_compressed(os.path.join(HERE, "qembed_cases.npz"), **make_qembed(rng))
    np.savez_compressed(os.path.join(HERE, "quantize_cases.npz"), **make_quantize(rng))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
