"""Bit-exact parity of the HIP masked gathers, quantizer and dequantizer with the oracle."""
import os

import numpy as np
import pytest
import torch

from oracle.bf16 import f32_to_bf16
from oracle.gather import qembed_gather_bf16, vocab_gather_bf16
from oracle.mlx_affine import dequantize_bf16, quantize_bf16
from shardcompute_amd import _lib
from tests.gpu_util import dev, dev_bf16, dev_u32, host_u16, host_u32

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _gather(ids, table, start):
    out = _lib.vocab_gather(dev(ids), dev_bf16(table), start)
    torch.cuda.synchronize()
    return host_u16(out)


def test_gather_golden(device):
    z = np.load(os.path.join(GOLD, "gather_cases.npz"), allow_pickle=False)
    for ids, table, start, out in (("ids", "table", "start", "out"), ("vids", "vtable", "vstart", "vout"),
                                   ("oids", "otable", "ostart", "oout")):
        print(f"gather golden {ids}", flush=True)
        got = _gather(z[ids], z[table], int(z[start]))
        assert np.array_equal(got, z[out])


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_gather_edges(device, dtype):
    rng = np.random.default_rng(1)
    V, D, start = 300, 4096, 300
    table = f32_to_bf16(rng.standard_normal((V, D)).astype(np.float32))
    table[5, :3] = [0x8000, 0x7FC1, 0xFF80]
    ids = np.array([start - 1, start, start + 5, start + V - 1, start + V, -1, 2 ** 31 - 1 if dtype == np.int32
                    else 2 ** 40, -(2 ** 31)], dtype=dtype)
    assert np.array_equal(_gather(ids, table, start), vocab_gather_bf16(ids, table, start))
    empty = _lib.vocab_gather(dev(np.zeros((0,), dtype)), dev_bf16(table), start)
    assert tuple(empty.shape) == (0, D)


def _zipf_ids(rng, shape, vocab, s=1.1):
    p = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    p /= p.sum()
    return rng.choice(vocab, size=shape, p=p).astype(np.int64)


@pytest.mark.parametrize("rank", [0, 1])
def test_gather_vocab_sharded_full_size(device, rank):
    """Rank `rank` of a world_size-2 split of a 128256 x 4096 bf16 table, Zipf(1.1) ids [64, 2048]."""
    rng = np.random.default_rng(0)
    V, D, ws = 128256, 4096, 2
    vl = V // ws
    start = rank * vl
    ids = _zipf_ids(rng, (64, 2048), V)
    table = torch.randn(vl, D, generator=torch.Generator().manual_seed(rank), dtype=torch.float32) * 0.02
    table_u16 = table.bfloat16().view(torch.int16).numpy().view(np.uint16)
    tdev = dev_bf16(table_u16)
    out = _lib.vocab_gather(dev(ids), tdev, start)
    torch.cuda.synchronize()
    for b0 in range(0, 64, 8):
        print(f"full-size gather rank={rank} rows {b0}..{b0 + 8}", flush=True)
        got = host_u16(out[b0:b0 + 8])
        assert np.array_equal(got, vocab_gather_bf16(ids[b0:b0 + 8], table_u16, start))


def test_gather_shards_sum_to_full_lookup(device):
    """Summing every rank's masked rows gives the unsharded lookup (the all-reduce identity)."""
    rng = np.random.default_rng(2)
    V, D, ws = 1024, 256, 4
    full = f32_to_bf16(rng.standard_normal((V, D)).astype(np.float32))
    ids = rng.integers(0, V, size=(3, 50)).astype(np.int32)
    acc = None
    for r in range(ws):
        part = _lib.vocab_gather(dev(ids), dev_bf16(full[r * V // ws:(r + 1) * V // ws]), r * V // ws).float()
        acc = part if acc is None else acc + part
    ref = _lib.vocab_gather(dev(ids), dev_bf16(full), 0).float()
    assert torch.equal(acc, ref)


@pytest.mark.parametrize("bits", [4, 8])
def test_qembed_golden_and_random(device, bits):
    z = np.load(os.path.join(GOLD, "qembed_cases.npz"), allow_pickle=False)
    p = f"w{bits}_"
    got = _lib.qembed_gather(dev(z[p + "ids"]), dev_u32(z[p + "wq"]), dev_bf16(z[p + "s"]), dev_bf16(z[p + "b"]),
                             int(z["start"]), bits)
    assert np.array_equal(host_u16(got), z[p + "out"])
    rng = np.random.default_rng(bits)
    V, D, start = 2000, 4096, 2000
    wq, s, b = quantize_bf16((rng.standard_normal((V, D)) * 0.02).astype(np.float32), 64, bits)
    ids = rng.integers(0, 6000, size=(4, 100)).astype(np.int32)
    got = _lib.qembed_gather(dev(ids), dev_u32(wq), dev_bf16(s), dev_bf16(b), start, bits)
    assert np.array_equal(host_u16(got), qembed_gather_bf16(ids, wq, s, b, start, 64, bits))


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_bit_exact(device, bits):
    z = np.load(os.path.join(GOLD, "quantize_cases.npz"), allow_pickle=False)
    wq, s, b = _lib.quantize(dev(z["w"]), bits)
    assert np.array_equal(host_u32(wq), z[f"wq{bits}"])
    assert np.array_equal(host_u16(s), z[f"s{bits}"]) and np.array_equal(host_u16(b), z[f"b{bits}"])
    rng = np.random.default_rng(3 + bits)
    w = (rng.standard_normal((512, 4096)) * 0.02).astype(np.float32)
    wq, s, b = _lib.quantize(dev(w), bits)
    rq, rs, rb = quantize_bf16(w, 64, bits)
    assert np.array_equal(host_u32(wq), rq)
    assert np.array_equal(host_u16(s), rs) and np.array_equal(host_u16(b), rb)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_bit_exact(device, bits):
    rng = np.random.default_rng(11)
    wq, s, b = quantize_bf16((rng.standard_normal((300, 1024)) * 0.02).astype(np.float32), 64, bits)
    got = _lib.dequantize(dev_u32(wq), dev_bf16(s), dev_bf16(b), bits)
    assert np.array_equal(host_u16(got), dequantize_bf16(wq, s, b, 64, bits))
