"""GPU parity of the decoder-wiring kernels with the oracle restatement.

* RMSNorm (+ fused residual add): the residual sum is bit-exact; the normalised
  output is within 1 bf16 step (the fp32 sum of squares is reduced in a
  different order than numpy's pairwise mean).
* RoPE + KV append: bit-exact (same fp32 tables, same unfused op order).
* Attention: max-abs-rel <= 1e-2 against the fp32 oracle (the kernel feeds the
  probabilities to the second product as bf16), over decode (split keys),
  prefill, chunked prefill, GQA ratios 1..32 and head_dim 64/128, with finite
  garbage past the cache length to prove masking.
* SiLU gate: within 1 bf16 step (device expf vs numpy exp).
* argmax: exact first-max index including ties, NaN and signed zeros.
"""
import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16, round_bf16
from oracle.decoder import apply_rope, attention_core, rms_norm, rope_cos_sin
from shardcompute_amd import _lib
from shardcompute_amd.parallel.attention import rope_tables_np
from tests.gpu_util import bf16_ulp_diff, dev, dev_bf16, host_u16

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-2


def _bf(rng, shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("rows,D", [(1, 4096), (5, 2048), (3, 64), (2, 8192), (4, 14336)])
def test_rms_norm(device, rows, D):
    rng = np.random.default_rng(rows * 1000 + D)
    x, r = _bf(rng, (rows, D)), _bf(rng, (rows, D))
    w = f32_to_bf16((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    eps = 1e-5
    h_ref = f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(r))
    y_ref = f32_to_bf16(rms_norm(bf16_to_f32(h_ref), w, eps))
    y0_ref = f32_to_bf16(rms_norm(bf16_to_f32(x), w, eps))
    xd, rd, wd = dev_bf16(x), dev_bf16(r), dev_bf16(w)
    h = torch.empty_like(xd)
    y = _lib.rms_norm(xd, wd, eps, residual=rd, h_out=h)
    y0 = _lib.rms_norm(xd, wd, eps)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(h), h_ref)
    for got, ref in ((host_u16(y), y_ref), (host_u16(y0), y0_ref)):
        d = bf16_ulp_diff(got, ref)
        assert d.max() <= 1, d.max()
        assert (d > 0).mean() < 0.01


def test_rms_norm_in_place_residual(device):
    rng = np.random.default_rng(7)
    x, r = _bf(rng, (3, 4096)), _bf(rng, (3, 4096))
    w = f32_to_bf16(np.ones(4096, np.float32))
    h_ref = f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(r))
    xd = dev_bf16(x)
    _lib.rms_norm(xd, dev_bf16(w), 1e-5, residual=dev_bf16(r), h_out=xd)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(xd), h_ref)


def test_rms_norm_constant_rows(device):
    # closed form: a constant row c normalises to sign(c) * w / sqrt(1 + eps / c^2)
    D = 1024
    c = np.array([0.5, -2.0, 3.0], np.float32)
    x = f32_to_bf16(np.repeat(c[:, None], D, 1))
    w = f32_to_bf16(np.linspace(0.5, 1.5, D).astype(np.float32))
    y = host_u16(_lib.rms_norm(dev_bf16(x), dev_bf16(w), 0.0))
    expect = f32_to_bf16(np.sign(c)[:, None] * bf16_to_f32(w)[None, :])
    assert np.array_equal(y, expect)


@pytest.mark.parametrize("B,S,H,Hkv,D,past,offset", [
    (1, 1, 32, 8, 128, 2047, 0),
    (2, 7, 8, 2, 64, 0, 0),
    (1, 33, 4, 4, 128, 100, 0),
    (3, 2, 8, 1, 128, 5, 1000),
    (2, 100, 8, 2, 64, 37, 5),         # many positions: v through the 64-token transpose
    (1, 300, 32, 8, 128, 1000, 0),
])
def test_rope_append(device, B, S, H, Hkv, D, past, offset):
    rng = np.random.default_rng(B + S + H + past)
    T_cap = ((past + S + 31) // 32) * 32
    width = (H + 2 * Hkv) * D + 24   # row stride wider than the heads
    rows = _bf(rng, (B * S, width))
    base = 500000.0
    cos_h, sin_h = rope_tables_np(D, base, 1.0, T_cap + offset + 8)
    oc, os_ = rope_cos_sin(np.arange(T_cap + offset + 8), D, base)
    assert np.array_equal(cos_h, oc[:, :D // 2]) and np.array_equal(sin_h, os_[:, :D // 2])
    qkv = dev_bf16(rows)
    kc = torch.zeros((B, Hkv, T_cap, D), dtype=torch.bfloat16, device="cuda")
    vt = torch.zeros((B, Hkv, D, T_cap), dtype=torch.bfloat16, device="cuda")
    cnt = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    _lib.rope_append_kv(qkv, B, S, H, Hkv, D, dev(cos_h), dev(sin_h), kc, vt, cnt, pos_offset=offset)
    torch.cuda.synchronize()
    pos = past + offset + np.arange(S)
    cos, sin = rope_cos_sin(pos, D, base)
    r32 = bf16_to_f32(rows)
    q = r32[:, :H * D].reshape(B, S, H, D).transpose(0, 2, 1, 3)
    k = r32[:, H * D:(H + Hkv) * D].reshape(B, S, Hkv, D).transpose(0, 2, 1, 3)
    v = rows[:, (H + Hkv) * D:(H + 2 * Hkv) * D].reshape(B, S, Hkv, D).transpose(0, 2, 1, 3)
    q_ref = f32_to_bf16(apply_rope(q, cos, sin)).transpose(0, 2, 1, 3).reshape(B * S, H * D)
    k_ref = f32_to_bf16(apply_rope(k, cos, sin))
    got = host_u16(qkv)
    assert np.array_equal(got[:, :H * D], q_ref)
    assert np.array_equal(got[:, H * D:], rows[:, H * D:])          # k, v and padding untouched
    kh, vh = host_u16(kc), host_u16(vt)
    assert np.array_equal(kh[:, :, past:past + S], k_ref)
    assert np.array_equal(vh[:, :, :, past:past + S], v.transpose(0, 1, 3, 2))
    mask = np.ones(T_cap, bool)
    mask[past:past + S] = False
    assert not kh[:, :, mask].any() and not vh[:, :, :, mask].any()


def _attn_case(rng, B, S, H, Hkv, D, past, extra_cap=0, nan_past=False):
    T = past + S
    T_cap = ((T + extra_cap + 31) // 32) * 32
    q = _bf(rng, (B * S, H * D))
    k = _bf(rng, (B, Hkv, T_cap, D))          # finite garbage past T must be masked out
    v = _bf(rng, (B, Hkv, T_cap, D))
    if nan_past:                              # slots past T may hold anything, NaN included
        k[:, :, T:] = 0x7FC0
        v[:, :, T:] = 0x7FC0
    kc = dev_bf16(k)
    vt = dev_bf16(np.ascontiguousarray(v.transpose(0, 1, 3, 2)))
    cnt = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    out = _lib.attention(dev_bf16(q), B, S, H, Hkv, D, kc, vt, cnt, 1.0 / np.sqrt(D))
    torch.cuda.synchronize()
    rep = H // Hkv
    q4 = bf16_to_f32(q).reshape(B, S, H, D).transpose(0, 2, 1, 3)
    kk = np.repeat(bf16_to_f32(k[:, :, :T]), rep, axis=1)
    vv = np.repeat(bf16_to_f32(v[:, :, :T]), rep, axis=1)
    ref = attention_core(q4, kk, vv, 1.0 / np.sqrt(D), T - S).transpose(0, 2, 1, 3).reshape(B * S, H * D)
    got = bf16_to_f32(host_u16(out))
    err = np.abs(got - ref).max() / np.abs(ref).max()
    return err


@pytest.mark.parametrize("B,S,H,Hkv,D,past,extra", [
    (1, 1, 32, 8, 128, 2047, 256),    # Llama-3-8B decode, split keys
    (1, 1, 32, 8, 128, 0, 0),         # first position
    (1, 1, 32, 4, 64, 150, 4000),     # TinyLlama decode, mostly empty splits
    (16, 1, 32, 8, 128, 300, 0),      # batch-16 decode
    (4, 1, 8, 1, 128, 1023, 0),       # 70B rank-0 shard heads, batch 4
    (1, 1, 32, 1, 64, 70, 0),         # 32 heads on one KV head (two head groups)
    (1, 1, 6, 6, 128, 40, 0),         # no GQA
    (1, 64, 32, 8, 128, 0, 0),        # prefill
    (2, 77, 8, 2, 64, 0, 5),          # ragged prefill, batch 2
    (1, 48, 32, 8, 128, 200, 0),      # chunked prefill after a cache
    (1, 5, 12, 4, 64, 3, 0),          # 3 heads per KV head (16 columns not filled)
    # long prefills (128-column workgroups)
    (1, 512, 32, 8, 128, 0, 0),       # Llama-3-8B heads
    (1, 512, 32, 8, 128, 700, 64),    # after a cache, the length off the block grid
    (1, 640, 32, 32, 128, 0, 0),      # no GQA: 128 positions of one head a workgroup
    (2, 300, 64, 8, 128, 17, 0),      # 70B heads (8 per KV head), ragged, batch 2
    (8, 130, 16, 2, 128, 0, 100),     # 8 heads per KV head, batch 8, a last block of 2 positions
])
def test_attention(device, B, S, H, Hkv, D, past, extra):
    rng = np.random.default_rng(B * 7 + S * 13 + H + past)
    err = _attn_case(rng, B, S, H, Hkv, D, past, extra)
    print(f"attention B={B} S={S} H={H} Hkv={Hkv} D={D} past={past}: max-abs-rel {err:.2e}", flush=True)
    assert err <= ATTN_TOL


@pytest.mark.parametrize("growth", ["steep", "gentle"])
def test_attention_prefill_running_max(device, growth):
    # the 128-column kernel moves a column's running maximum only when it grew by more
    # than 2^8 in probability: keys whose scores grow along the sequence make it move
    # often ("steep": e^10 per 64-key block) or stay put with probabilities near 256
    # ("gentle": 5.5 bits over the whole sequence); both must match the reference
    B, S, H, Hkv, D = 1, 512, 32, 8, 128
    rng = np.random.default_rng(17 if growth == "steep" else 18)
    T_cap = S
    q = rng.standard_normal((B * S, H * D)).astype(np.float32) * 0.5
    k = rng.standard_normal((B, Hkv, T_cap, D)).astype(np.float32) * 0.5
    # a shared direction in q and k whose weight grows with the key's position
    dirv = rng.standard_normal(D).astype(np.float32)
    dirv /= np.linalg.norm(dirv)
    per_key = 10.0 / 64 if growth == "steep" else 5.5 * np.log(2) / S
    scale = 1.0 / np.sqrt(D)
    q += np.tile(dirv, H)[None, :] * 4.0
    k += (np.arange(T_cap, dtype=np.float32)[:, None] * per_key / (4.0 * scale)) * dirv[None, :]
    q, k = f32_to_bf16(q), f32_to_bf16(k)
    v = _bf(rng, (B, Hkv, T_cap, D))
    cnt = torch.tensor([0, 0], dtype=torch.int32, device="cuda")
    out = _lib.attention(dev_bf16(q), B, S, H, Hkv, D, dev_bf16(k),
                         dev_bf16(np.ascontiguousarray(v.transpose(0, 1, 3, 2))), cnt, scale)
    torch.cuda.synchronize()
    rep = H // Hkv
    q4 = bf16_to_f32(q).reshape(B, S, H, D).transpose(0, 2, 1, 3)
    kk = np.repeat(bf16_to_f32(k), rep, axis=1)
    vv = np.repeat(bf16_to_f32(v), rep, axis=1)
    ref = attention_core(q4, kk, vv, scale, 0).transpose(0, 2, 1, 3).reshape(B * S, H * D)
    got = bf16_to_f32(host_u16(out))
    err = np.abs(got - ref).max() / np.abs(ref).max()
    print(f"attention, running maximum {growth}: max-abs-rel {err:.2e}", flush=True)
    assert np.isfinite(got).all() and err <= ATTN_TOL


@pytest.mark.parametrize("B,S,H,Hkv,D,past,extra", [
    (1, 48, 32, 8, 128, 200, 40),     # 16-column workgroups
    (1, 300, 32, 8, 64, 17, 40),      # head_dim 64
    (1, 512, 32, 8, 128, 0, 40),      # 128-column workgroups
    (1, 640, 32, 8, 128, 250, 70),    # 128-column workgroups, the length inside a block
])
def test_attention_nan_past_length(device, B, S, H, Hkv, D, past, extra):
    # cache slots at or past the length hold NaN: they must not reach the output
    rng = np.random.default_rng(S + past)
    err = _attn_case(rng, B, S, H, Hkv, D, past, extra, nan_past=True)
    print(f"attention (NaN past T) B={B} S={S} H={H} Hkv={Hkv} D={D} past={past}: max-abs-rel {err:.2e}", flush=True)
    assert np.isfinite(err) and err <= ATTN_TOL


def _mask_for(rng, kind, B, H, S, T):
    """An additive mask of the named layout, key 0 always visible (finite rows)."""
    if kind == "pad":                       # [B, 1, 1, T]: some keys hidden per sequence
        m = np.zeros((B, 1, 1, T), np.float32)
        for b in range(B):
            hide = rng.choice(np.arange(1, T), size=max(1, T // 5), replace=False)
            m[b, 0, 0, hide] = -np.inf
        return m
    if kind == "full":                      # [B, H, S, T]
        m = rng.standard_normal((B, H, S, T)).astype(np.float32) * 2
        m[..., 1::7] = -np.inf
        return m
    if kind == "rowcol":                    # [S, T]: leading dimensions broadcast
        return (rng.standard_normal((S, T)) * 1.5).astype(np.float32)
    if kind == "padmin":                    # [B, 1, S, T]: left padding with finfo(float32).min
        # sequence b's first pad[b] keys are padding; its padded query rows (prefill from
        # position 0) see only padding keys, so every visible key of such a row carries
        # finfo.min: the reference's softmax gives them uniform weights (finite rows)
        m = np.zeros((B, 1, S, T), np.float32)
        for b in range(B):
            pad = 3 + 7 * b
            m[b, 0, :, :pad] = np.finfo(np.float32).min
        return m
    if kind == "allmin":                    # [B, 1, S, T]: every key finfo(float32).min
        return np.full((B, 1, S, T), np.finfo(np.float32).min, np.float32)
    raise ValueError(kind)


@pytest.mark.parametrize("B,S,H,Hkv,D,past,extra,kind", [
    (2, 64, 32, 8, 128, 0, 0, "pad"),       # prefills: the 128-column kernel with the mask added
    (1, 160, 32, 8, 128, 64, 32, "full"),   # a per-head mask after a cached prefix
    (2, 96, 8, 1, 128, 0, 0, "padmin"),     # 8 q heads per kv head, left padding with finfo.min
    (1, 64, 32, 8, 128, 0, 0, "allmin"),    # every key finfo.min: uniform weights
    (1, 48, 8, 2, 64, 100, 30, "full"),     # head_dim 64, after a cache
    (1, 1, 32, 8, 128, 2047, 256, "pad"),   # one position, keys split over workgroups
    (3, 1, 8, 1, 128, 300, 0, "full"),      # one position, 8 heads per KV head
    (1, 200, 32, 8, 128, 0, 40, "rowcol"),
    (2, 64, 32, 8, 128, 0, 0, "padmin"),    # rows masked everywhere with finfo.min: uniform
    (1, 1, 32, 8, 128, 300, 0, "allmin"),   # one position, every key finfo.min, split ranges
    (2, 40, 8, 2, 64, 20, 8, "allmin"),     # after a cache: the causal limit still applies
])
def test_attention_additive_mask(device, B, S, H, Hkv, D, past, extra, kind):
    rng = np.random.default_rng(B + S + past)
    T = past + S
    T_cap = ((T + extra + 31) // 32) * 32
    q = _bf(rng, (B * S, H * D))
    k = _bf(rng, (B, Hkv, T_cap, D))
    v = _bf(rng, (B, Hkv, T_cap, D))
    m = _mask_for(rng, kind, B, H, S, T)
    cnt = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    print(f"attention with a {kind} mask {m.shape}: B={B} S={S} H={H} Hkv={Hkv} D={D} past={past}", flush=True)
    out = _lib.attention(dev_bf16(q), B, S, H, Hkv, D, dev_bf16(k),
                         dev_bf16(np.ascontiguousarray(v.transpose(0, 1, 3, 2))), cnt, 1.0 / np.sqrt(D),
                         mask=torch.from_numpy(m).cuda(), n_keys=T)
    torch.cuda.synchronize()
    rep = H // Hkv
    q4 = bf16_to_f32(q).reshape(B, S, H, D).transpose(0, 2, 1, 3)
    kk = np.repeat(bf16_to_f32(k[:, :, :T]), rep, axis=1)
    vv = np.repeat(bf16_to_f32(v[:, :, :T]), rep, axis=1)
    ref = attention_core(q4, kk, vv, 1.0 / np.sqrt(D), T - S, mask=m).transpose(0, 2, 1, 3).reshape(B * S, H * D)
    got = bf16_to_f32(host_u16(out))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() / np.abs(ref).max() <= ATTN_TOL


def test_attention_mask_errors(device):
    q = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, 2, 32, 128), dtype=torch.bfloat16, device="cuda")
    vt = torch.zeros((1, 2, 128, 32), dtype=torch.bfloat16, device="cuda")
    cnt = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="does not broadcast"):
        _lib.attention(q, 1, 4, 2, 2, 128, kc, vt, cnt, 0.1, mask=torch.zeros((1, 3, 4, 4), device="cuda"),
                       n_keys=4)
    with pytest.raises(ValueError, match="n_keys"):
        _lib.attention(q, 1, 4, 2, 2, 128, kc, vt, cnt, 0.1, mask=torch.zeros((4, 4), device="cuda"))


def _decode_case(rng, B, H, Hkv, D, past, T_cap, offset=0, base=500000.0):
    width = (H + 2 * Hkv) * D + 40                  # row stride wider than the heads
    rows = _bf(rng, (B, width))
    k = _bf(rng, (B, Hkv, T_cap, D))                # finite garbage past the cached keys
    v = _bf(rng, (B, Hkv, T_cap, D))
    cos_h, sin_h = rope_tables_np(D, base, 1.0, T_cap + offset)
    return rows, k, v, dev(cos_h), dev(sin_h)


@pytest.mark.parametrize("B,H,Hkv,D,past,extra,offset", [
    (1, 32, 8, 128, 2047, 256, 0),    # Llama-3-8B decode: split keys, merged by the last range
    (1, 32, 8, 128, 0, 0, 0),         # first position: only the new key
    (1, 32, 8, 128, 127, 2000, 0),    # the new key opens a range of its own
    (1, 32, 8, 128, 31, 0, 0),        # the new key at a block boundary
    (1, 32, 4, 64, 150, 4000, 0),     # TinyLlama heads, mostly empty ranges
    (16, 32, 8, 128, 300, 0, 0),      # batch 16
    (4, 8, 1, 128, 1023, 0, 0),       # 70B rank-0 shard heads, batch 4
    (1, 6, 6, 128, 40, 0, 0),         # no GQA
    (2, 8, 2, 64, 5, 0, 1000),        # rotary offset (cache-less calls)
])
def test_attention_decode_matches_two_kernel_path(device, B, H, Hkv, D, past, extra, offset):
    rng = np.random.default_rng(B * 11 + H + past + extra)
    T_cap = ((past + 1 + extra + 31) // 32) * 32
    rows, k, v, cos_t, sin_t = _decode_case(rng, B, H, Hkv, D, past, T_cap, offset)
    vt_h = np.ascontiguousarray(v.transpose(0, 1, 3, 2))
    scale = 1.0 / np.sqrt(D)
    print(f"attention_decode B={B} H={H} Hkv={Hkv} D={D} past={past} T_cap={T_cap} offset={offset}", flush=True)
    # fused
    kc1, vt1 = dev_bf16(k), dev_bf16(vt_h)
    cnt1 = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    qkv1 = dev_bf16(rows)
    ws = torch.empty(max(_lib.attention_decode_workspace_bytes(B, H, Hkv, D, T_cap), 16), dtype=torch.uint8,
                     device="cuda")
    out1 = _lib.attention_decode(qkv1, B, H, Hkv, D, cos_t, sin_t, kc1, vt1, cnt1, scale, pos_offset=offset,
                                 workspace=ws)
    # two kernels
    kc2, vt2 = dev_bf16(k), dev_bf16(vt_h)
    cnt2 = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    qkv2 = dev_bf16(rows)
    _lib.rope_append_kv(qkv2, B, 1, H, Hkv, D, cos_t, sin_t, kc2, vt2, cnt2, pos_offset=offset)
    out2 = _lib.attention(qkv2, B, 1, H, Hkv, D, kc2, vt2, cnt2, scale)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vt1, vt2)           # same cache contents
    assert torch.equal(qkv1, dev_bf16(rows))                        # the q|k|v row is not modified
    a, b = bf16_to_f32(host_u16(out1)), bf16_to_f32(host_u16(out2))
    assert np.abs(a - b).max() <= 1e-2 * np.abs(b).max()
    # against the oracle: rotated q and the cache after the append
    T = past + 1
    kh = bf16_to_f32(host_u16(kc1)[:, :, :T])
    vh = bf16_to_f32(host_u16(vt1)[:, :, :, :T]).transpose(0, 1, 3, 2)
    cos, sin = rope_cos_sin(np.array([past + offset]), D, 500000.0)
    q = bf16_to_f32(rows[:, :H * D]).reshape(B, 1, H, D).transpose(0, 2, 1, 3)
    q = bf16_to_f32(f32_to_bf16(apply_rope(q, cos, sin)))
    rep = H // Hkv
    ref = attention_core(q, np.repeat(kh, rep, axis=1), np.repeat(vh, rep, axis=1), scale, T - 1)
    ref = ref.transpose(0, 2, 1, 3).reshape(B, H * D)
    assert np.abs(a - ref).max() / np.abs(ref).max() <= ATTN_TOL


def test_attention_decode_graph_replays(device):
    # captured once, replayed with the cache length advancing on the device; every
    # replay equals the eager two-kernel path at that length
    B, H, Hkv, D, past, T_cap = 1, 32, 8, 128, 500, 1024
    rng = np.random.default_rng(77)
    rows, k, v, cos_t, sin_t = _decode_case(rng, B, H, Hkv, D, past, T_cap)
    vt_h = np.ascontiguousarray(v.transpose(0, 1, 3, 2))
    scale = 1.0 / np.sqrt(D)
    kc1, vt1 = dev_bf16(k), dev_bf16(vt_h)
    kc2, vt2 = dev_bf16(k), dev_bf16(vt_h)
    cnt1 = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    qkv1 = dev_bf16(rows)
    ws = torch.empty(max(_lib.attention_decode_workspace_bytes(B, H, Hkv, D, T_cap), 16), dtype=torch.uint8,
                     device="cuda")
    out1 = torch.empty((B, H * D), dtype=torch.bfloat16, device="cuda")
    _lib.attention_decode(qkv1, B, H, Hkv, D, cos_t, sin_t, kc1, vt1, cnt1, scale, out=out1, workspace=ws)
    _lib.add_i32(cnt1, 1, n=1)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.attention_decode(qkv1, B, H, Hkv, D, cos_t, sin_t, kc1, vt1, cnt1, scale, out=out1, workspace=ws)
        _lib.add_i32(cnt1, 1, n=1)
    cnt2 = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    for step in range(4):
        qkv2 = dev_bf16(rows)
        _lib.rope_append_kv(qkv2, B, 1, H, Hkv, D, cos_t, sin_t, kc2, vt2, cnt2, pos_offset=0)
        ref = _lib.attention(qkv2, B, 1, H, Hkv, D, kc2, vt2, cnt2, scale)
        _lib.add_i32(cnt2, 1, n=1)
        if step > 0:
            g.replay()
        torch.cuda.synchronize()
        a, b = bf16_to_f32(host_u16(out1)), bf16_to_f32(host_u16(ref))
        assert np.abs(a - b).max() <= 1e-2 * np.abs(b).max(), step
        assert torch.equal(kc1, kc2) and torch.equal(vt1, vt2), step
    assert int(cnt1[0]) == past + 4


def test_attention_decode_errors(device):
    qkv = torch.zeros((1, 3 * 256), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, 2, 64, 128), dtype=torch.bfloat16, device="cuda")
    vt = torch.zeros((1, 2, 128, 64), dtype=torch.bfloat16, device="cuda")
    cnt = torch.zeros(2, dtype=torch.int32, device="cuda")
    c, s = torch.zeros((64, 64), device="cuda"), torch.zeros((64, 64), device="cuda")
    with pytest.raises(RuntimeError, match="16 q heads"):
        _lib.attention_decode(torch.zeros((1, 36 * 128), dtype=torch.bfloat16, device="cuda"), 1, 34, 1, 128, c, s,
                              torch.zeros((1, 1, 64, 128), dtype=torch.bfloat16, device="cuda"),
                              torch.zeros((1, 1, 128, 64), dtype=torch.bfloat16, device="cuda"), cnt, 0.1)
    with pytest.raises(ValueError, match="cos/sin"):
        _lib.attention_decode(qkv, 1, 2, 2, 128, c[:, :10], s[:, :10], kc, vt, cnt, 0.1)


def test_attention_single_key_is_value(device):
    # one cached position: softmax weight 1, output = v exactly (bf16 copy)
    B, S, H, Hkv, D = 1, 1, 8, 2, 128
    rng = np.random.default_rng(3)
    q = _bf(rng, (1, H * D))
    k = np.zeros((B, Hkv, 32, D), np.uint16)
    v = np.zeros((B, Hkv, 32, D), np.uint16)
    k[:, :, 0] = _bf(rng, (B, Hkv, D))
    v[:, :, 0] = _bf(rng, (B, Hkv, D))
    cnt = torch.tensor([0, 0], dtype=torch.int32, device="cuda")
    out = _lib.attention(dev_bf16(q), B, S, H, Hkv, D, dev_bf16(k),
                         dev_bf16(np.ascontiguousarray(v.transpose(0, 1, 3, 2))), cnt, 0.1)
    got = host_u16(out).reshape(H, D)
    assert np.array_equal(got, np.repeat(v[0, :, 0], H // Hkv, axis=0))


def test_attention_errors(device):
    q = torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, 2, 40, 128), dtype=torch.bfloat16, device="cuda")
    vt = torch.zeros((1, 2, 128, 40), dtype=torch.bfloat16, device="cuda")
    cnt = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 32"):
        _lib.attention(q, 1, 1, 2, 2, 128, kc, vt, cnt, 0.1)
    with pytest.raises(RuntimeError, match="head_dim"):
        _lib.attention(torch.zeros((1, 192), dtype=torch.bfloat16, device="cuda"), 1, 1, 2, 2, 96,
                       torch.zeros((1, 2, 32, 96), dtype=torch.bfloat16, device="cuda"),
                       torch.zeros((1, 2, 96, 32), dtype=torch.bfloat16, device="cuda"), cnt, 0.1)


@pytest.mark.parametrize("rows,I", [(1, 14336), (3, 5632), (2, 8)])
def test_silu_mul(device, rows, I):
    rng = np.random.default_rng(rows + I)
    gu = _bf(rng, (rows, 2 * I), 3.0)
    gu[0, :4] = [0x0000, 0x8000, 0x4120, 0xC120]        # 0, -0, 10, -10
    got = host_u16(_lib.silu_mul(dev_bf16(gu)))
    g, u = bf16_to_f32(gu[:, :I]), bf16_to_f32(gu[:, I:])
    ref = f32_to_bf16((g / (np.float32(1) + np.exp(-g, dtype=np.float32))) * u)
    d = bf16_ulp_diff(got, ref)
    assert d.max() <= 1
    assert (d > 0).mean() < 0.01


def test_argmax(device):
    rng = np.random.default_rng(11)
    V = 128256
    logits = _bf(rng, (6, V))
    logits[1, [10, 99, 5000]] = 0x4200             # ties at the maximum: first index wins
    logits[2, [7, 300]] = [0x7FC0, 0x7FC1]          # NaN counts as the maximum (first NaN)
    logits[3] = 0x8000                              # all -0.0 ...
    logits[3, 12] = 0x0000                          # ... and one +0.0: equal, index 0 wins
    logits[4] = 0xFF80                              # -inf everywhere but one -1e30
    logits[4, 77777] = 0xF149
    logits[5, [45, 41 + 8 * 1024, 41]] = 0x4300     # ties within one thread's elements
    ids = torch.empty(6, dtype=torch.int32, device="cuda")
    tokens = torch.full((6, 4), -1, dtype=torch.int32, device="cuda")
    step = torch.tensor([2], dtype=torch.int32, device="cuda")
    _lib.argmax(dev_bf16(logits), ids=ids, tokens=tokens, step=step)
    torch.cuda.synchronize()
    ref = np.argmax(bf16_to_f32(logits), axis=-1)
    assert np.array_equal(ids.cpu().numpy(), ref)
    assert ref[1] == 10 and ref[2] == 7 and ref[3] == 0 and ref[4] == 77777 and ref[5] == 41
    t = tokens.cpu().numpy()
    assert np.array_equal(t[:, 2], ref) and (t[:, [0, 1, 3]] == -1).all()
    # longer rows: a thread's elements span several load batches; a tie between two
    # batches of the same thread, and a lone maximum in the last batch
    big = _bf(rng, (3, 300000))
    big[1, [8 * (3 + 1024 * 33) + 1, 8 * (3 + 1024 * 20) + 5]] = 0x4300
    big[2, 299999] = 0x4300
    got = _lib.argmax(dev_bf16(big)).cpu().numpy()
    ref = np.argmax(bf16_to_f32(big), axis=-1)
    assert np.array_equal(got, ref) and ref[1] == 8 * (3 + 1024 * 20) + 5 and ref[2] == 299999
    # odd vocabulary (scalar path)
    small = _bf(rng, (3, 1001))
    got = _lib.argmax(dev_bf16(small)).cpu().numpy()
    assert np.array_equal(got, np.argmax(bf16_to_f32(small), axis=-1))


def test_add_and_counters(device):
    rng = np.random.default_rng(5)
    a, b = _bf(rng, (3, 4096)), _bf(rng, (3, 4096))
    got = host_u16(_lib.add(dev_bf16(a), dev_bf16(b)))
    assert np.array_equal(got, f32_to_bf16(bf16_to_f32(a) + bf16_to_f32(b)))
    c = torch.tensor([5, 9, 1], dtype=torch.int32, device="cuda")
    _lib.add_i32(c, 3, n=2)
    _lib.add_i32(c[2:], -1, n=1)
    assert c.cpu().tolist() == [8, 12, 0]


@pytest.mark.parametrize("B,H,Hkv,D,past,extra,kind", [
    (2, 32, 8, 128, 500, 64, "pad"),        # padding keys (-inf) in a long cache: split key ranges
    (3, 8, 1, 128, 300, 0, "full"),         # a per-head mask, 8 q heads per kv head
    (1, 32, 4, 64, 150, 100, "full"),       # head_dim 64
    (1, 32, 8, 128, 40, 0, "allmin"),       # every key finfo.min: uniform weights
    (2, 32, 8, 128, 64, 0, "newonly"),      # only the new key visible (the rest -inf)
])
def test_attention_decode_additive_mask(device, B, H, Hkv, D, past, extra, kind):
    """The fused decode attention with an additive mask against the oracle, the cache
    contents against the two-kernel path's, and the output against the masked
    two-kernel path (sc_rope_append_kv_bf16 then sc_attention_masked_bf16)."""
    rng = np.random.default_rng(B * 5 + H + past)
    T = past + 1
    T_cap = ((T + extra + 31) // 32) * 32
    rows, k, v, cos_t, sin_t = _decode_case(rng, B, H, Hkv, D, past, T_cap)
    vt_h = np.ascontiguousarray(v.transpose(0, 1, 3, 2))
    if kind == "newonly":
        m = np.full((B, 1, 1, T), -np.inf, np.float32)
        m[..., T - 1] = 0.0
    else:
        m = _mask_for(rng, kind, B, H, 1, T)
    mask = torch.from_numpy(m).cuda()
    scale = 1.0 / np.sqrt(D)
    print(f"attention_decode with a {kind} mask {m.shape}: B={B} H={H} Hkv={Hkv} D={D} past={past}", flush=True)
    ws = torch.empty(max(_lib.attention_decode_workspace_bytes(B, H, Hkv, D, T_cap),
                         _lib.attention_workspace_bytes(B, 1, H, Hkv, D, T_cap), 16), dtype=torch.uint8, device="cuda")
    kc1, vt1 = dev_bf16(k), dev_bf16(vt_h)
    cnt1 = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    out1 = _lib.attention_decode(dev_bf16(rows), B, H, Hkv, D, cos_t, sin_t, kc1, vt1, cnt1, scale, workspace=ws,
                                 mask=mask, n_keys=T)
    kc2, vt2 = dev_bf16(k), dev_bf16(vt_h)
    cnt2 = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    qkv2 = dev_bf16(rows)
    _lib.rope_append_kv(qkv2, B, 1, H, Hkv, D, cos_t, sin_t, kc2, vt2, cnt2)
    out2 = _lib.attention(qkv2, B, 1, H, Hkv, D, kc2, vt2, cnt2, scale, workspace=ws, mask=mask, n_keys=T)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vt1, vt2)
    a, b2 = bf16_to_f32(host_u16(out1)), bf16_to_f32(host_u16(out2))
    assert np.isfinite(a).all()
    assert np.abs(a - b2).max() <= 1e-2 * np.abs(b2).max()
    kh = bf16_to_f32(host_u16(kc1)[:, :, :T])
    vh = bf16_to_f32(host_u16(vt1)[:, :, :, :T]).transpose(0, 1, 3, 2)
    cos, sin = rope_cos_sin(np.array([past]), D, 500000.0)
    q = bf16_to_f32(rows[:, :H * D]).reshape(B, 1, H, D).transpose(0, 2, 1, 3)
    q = bf16_to_f32(f32_to_bf16(apply_rope(q, cos, sin)))
    rep = H // Hkv
    ref = attention_core(q, np.repeat(kh, rep, axis=1), np.repeat(vh, rep, axis=1), scale, T - 1, mask=m)
    ref = ref.transpose(0, 2, 1, 3).reshape(B, H * D)
    assert np.abs(a - ref).max() / np.abs(ref).max() <= ATTN_TOL


def test_attention_decode_mask_all_inf_row_is_nan(device):
    # every visible key -inf: 0 / 0, as the reference's softmax gives
    B, H, Hkv, D, past = 1, 8, 2, 128, 20
    rng = np.random.default_rng(9)
    rows, k, v, cos_t, sin_t = _decode_case(rng, B, H, Hkv, D, past, 64)
    mask = torch.full((1, 1, 1, past + 1), -float("inf"), device="cuda")
    cnt = torch.tensor([past, 0], dtype=torch.int32, device="cuda")
    out = _lib.attention_decode(dev_bf16(rows), B, H, Hkv, D, cos_t, sin_t, dev_bf16(k),
                                dev_bf16(np.ascontiguousarray(v.transpose(0, 1, 3, 2))), cnt, 0.1, mask=mask,
                                n_keys=past + 1)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
