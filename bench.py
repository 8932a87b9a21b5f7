#!/usr/bin/env python3
"""W4 g64 greedy decode throughput of a Llama-3-8B-shape decoder on one MI355X.

Workload: random-init Llama-3-8B shape (hidden 4096, intermediate 14336, 32
layers, 32 q / 8 kv heads of 128, vocab 128256, RoPE theta 500000, RMSNorm eps
1e-5), every linear N(0, 0.02) quantized to MLX affine 4-bit g64 on the GPU,
bf16 vocab embedding, W4 lm_head.  A 2048-token uniform-random prompt is
prefilled (timed separately, after one untimed prefill of the same shape), then
greedy decode runs as HIP-graph replays of 8 steps each.  A "step" is one decode token for the whole batch.

Printed (one JSON line on stdout):
* ``value``: decode tokens/s (batch x steps / wall time of the timed steps,
  bracketed by device synchronisation);
* ``roofline``: the dominant kernel of a decode step.  At batch 1 that is the
  whole-trunk launch ``decode_step_kernel<4, 128, 4>`` (embedding and every layer in one
  persistent kernel; the step adds the final RMSNorm + lm_head GEMV, which also
  selects the greedy token):
  algorithmic bytes per launch (every layer's packed weights + bf16 scales and
  biases, the KV cache read at the step's length, the appended key/value, the
  embedding row and the output row) over the average launch duration: HIP events
  on the launch stream around back-to-back launches, against 8 TB/s.  Without the
  trunk plan (batch > 1) it is the decode qGEMV, as ``qgemv_roofline``.
  ``traffic`` is the measured HBM bytes per launch recorded under ``profiles/``
  (null when absent);
* ``qgemv_roofline``: the per-op batch-1 decode qGEMV (``qgemv_m1_kernel<4, *, *>``,
  every prologue/epilogue instantiation: plain, RMSNorm, RMSNorm + SwiGLU) on the
  same weights: algorithmic bytes (packed weights + bf16 scales and biases + x + y)
  per launch, averaged over the 129 launches of one decode step, over the average
  launch duration (HIP events on the replay stream around graph replays of exactly
  those launches, so the average is the kernels' own), against 8 TB/s;
* ``cpu_baseline``: a CPU restatement of the quantized matmul, not MLX (MLX's CPU
  backend is not available; ``oracle/qmm_fast.c``: fp32 accumulation, AVX2 + FMA,
  OpenMP over this host's cores) timed on a bounded sample: decoder layer 0's four
  projections plus 1/32 of the lm_head rows at M = batch, repeated for ~10 s,
  scaled to tokens/s of the 32-layer model's linear layers;
* ``prefill.qgemm_roofline``: the prefill quantized GEMM at M = prompt tokens on
  layer 0's four projection shapes, TFLOP/s against 2.5 PFLOP/s dense bf16;
* ``other_configs``: the other workloads of the path, each beside the headline:
  the vocab-sharded gather of 64 x 2048 Zipf(1.1) ids on rank 0 of a 2-way split
  of the 128256 x 4096 table (GB/s on ids + written rows + unique in-shard rows
  read) and that configuration's W4 lm_head at M = 64; batch-16 decode of the
  headline model; the batch-1 decode qGEMV at 8 bits; TinyLlama-shape W4
  decode (32-token prompt, batch 1); the Llama-3-70B rank-0-of-8 shard at
  batch 32 after a 1024-token prefill, W4 and W8 (all-reduces as identity); and
  the standalone quantized-linear sweep (the six TinyLlama / Llama-3-8B
  projection shapes x M in {1, 8, 32, 512, 2048} x W4/W8, GPU time, GB/s or
  TFLOP/s and roofline fraction, beside the CPU restatement's time).
"""
import argparse
import asyncio
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "W4 decode tok/s (Llama-3-8B shape, bs1) + qGEMV HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.5e15
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qgemv_m1_w4_llama3_8b_decode_traffic.json")
TRUNK_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_step_w4_llama3_8b_traffic.json")

LLAMA3_8B = dict(vocab=128256, hidden=4096, inter=14336, layers=32, heads=32, kv_heads=8, theta=500000.0, eps=1e-5)
TINYLLAMA = dict(vocab=32000, hidden=2048, inter=5632, layers=22, heads=32, kv_heads=4, theta=10000.0, eps=1e-5)
LLAMA3_70B = dict(vocab=128256, hidden=8192, inter=28672, layers=80, heads=64, kv_heads=8, theta=500000.0, eps=1e-5)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128, help="timed decode steps")
    p.add_argument("--warmup", type=int, default=16, help="untimed decode steps")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--prefill", type=int, default=2048)
    p.add_argument("--layers", type=int, default=None, help="decoder layers (default: the model's)")
    p.add_argument("--model", choices=("llama3-8b", "tinyllama"), default="llama3-8b",
                   help="decoder shape of the headline run (the JSON line is the Llama-3-8B one; tinyllama is "
                        "for the timeline and kernel-only diagnostics)")
    p.add_argument("--bits", type=int, default=4, choices=(4, 8))
    p.add_argument("--kernel-reps", type=int, default=5, help="graph replays of the per-launch GEMV timing")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--kernels-only", action="store_true",
                   help="build the weights and run only the per-launch GEMV pass (for counter profiling)")
    p.add_argument("--gemm-only", action="store_true",
                   help="build the weights and run only the prefill quantized GEMM timing (for counter profiling)")
    p.add_argument("--attn-only", action="store_true",
                   help="run only the prefill attention of the Llama-3-8B heads at --prefill positions "
                        "(random q, k, v; for counter profiling)")
    p.add_argument("--batched-decode-only", action="store_true",
                   help="only the batched decode workloads: Llama-3-8B at batch 16 and the 70B rank-0 shard at "
                        "batch 32, W4 (one JSON line)")
    p.add_argument("--shard-head-only", action="store_true",
                   help="only the vocab-sharded embedding gather and the M=64 quantized lm_head (one JSON line)")
    p.add_argument("--sweep-only", action="store_true",
                   help="only the standalone quantized-linear sweep (every (K, N), M, W4/W8), JSON on stdout")
    p.add_argument("--gemv16-only", action="store_true",
                   help="run only the 9-32-row quantized GEMV on the batched-decode projection shapes "
                        "(70B rank-0 shard at 32 rows, Llama-3-8B at 16; for counter profiling)")
    p.add_argument("--trunk-only", action="store_true",
                   help="prefill, then only eager whole-trunk decode launches (for counter profiling)")
    p.add_argument("--trunk-timeline", action="store_true",
                   help="prefill, then print the whole-trunk launch's per-op timeline (JSON) and exit")
    p.add_argument("--no-extras", dest="extras", action="store_false",
                   help="skip the other configurations' measurements (gather, lm_head, batch 16, W8, ...)")
    p.add_argument("--no-extra-models", dest="extras_models", action="store_false",
                   help="skip the extra model builds (W8 GEMV, TinyLlama, 70B shard)")
    return p.parse_args()


# ---------------------------------------------------------------- model


def build_model(cfg, layers, bits, capacity, seed=0, world_size=1, rank=0):
    """Random-init quantized decoder of shape ``cfg``; with world_size > 1, rank
    ``rank``'s shard (local heads, intermediate and vocab rows), its collectives
    the identity."""
    import torch
    from shardcompute_amd import _lib
    from shardcompute_amd.communicator import IdentityCommunicator
    from shardcompute_amd.parallel.transformer import ParallelTransformer
    dev = torch.device("cuda", 0)
    ws = world_size
    H, I, V = cfg["hidden"], cfg["inter"], cfg["vocab"]
    D = H // cfg["heads"]
    nq, nkv = cfg["heads"] // ws * D, cfg["kv_heads"] // ws * D
    I, V = I // ws, V // ws
    comm = IdentityCommunicator(rank, ws) if ws > 1 else None
    m = ParallelTransformer(vocab_size=cfg["vocab"], hidden_size=H, num_layers=layers, num_heads=cfg["heads"],
                            intermediate_size=cfg["inter"], world_size=ws, rank=rank, communicator=comm,
                            num_kv_heads=cfg["kv_heads"], max_position_embeddings=capacity,
                            rms_norm_eps=cfg["eps"], rope_base=cfg["theta"], use_quantized=True,
                            quantization_bits=bits, quantization_group_size=64, embedding="vocab",
                            quantized_lm_head=True, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def q(n, k):
        w = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32).mul_(0.02)
        out = _lib.quantize(w, bits=bits)
        del w
        return out

    def norm_w():
        return (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)

    for layer in m.layers:
        layer.input_layernorm.load_weights(norm_w())
        layer.post_attention_layernorm.load_weights(norm_w())
        wq, s, b = q(nq + 2 * nkv, H)
        o = q(H, nq)
        sl = [slice(0, nq), slice(nq, nq + nkv), slice(nq + nkv, nq + 2 * nkv)]
        layer.attention.load_quantized_shards(wq[sl[0]], s[sl[0]], b[sl[0]], None, wq[sl[1]], s[sl[1]], b[sl[1]],
                                              None, wq[sl[2]], s[sl[2]], b[sl[2]], None, *o, None)
        gwq, gs, gb = q(2 * I, H)
        d = q(H, I)
        layer.mlp.load_quantized_shards(gwq[I:], gs[I:], gb[I:], None, *d, None, gwq[:I], gs[:I], gb[:I], None)
        del wq, s, b, gwq, gs, gb
    emb = torch.randn((V, H), generator=g, device=dev, dtype=torch.float32).mul_(0.02).to(torch.bfloat16)
    m.load_embedding_weights(emb)
    m.load_norm_weights(norm_w())
    m.load_quantized_lm_head_weights(*q(V, H))
    # build the fused q|k|v and gate|up matrices now (outside any timed region)
    for layer in m.layers:
        layer.attention.qkv.build()
        layer.mlp.gate_up.build()
    torch.cuda.synchronize()
    return m


def gemv_launches(model):
    """(name, prologue, wq, scales, biases, K, N) of every quantized product of one
    decode step, with the transformations its kernel applies: "norm" (RMSNorm +
    residual add on the input), "norm+swiglu" (and silu(gate) * up on paired output
    columns) or "" (plain)."""
    out = []
    for layer in model.layers:
        att, mlp = layer.attention, layer.mlp
        qkv, gu = att.qkv, mlp.gate_up
        K = model.hidden_size
        out.append(("qkv", "norm", qkv._wq, qkv._s, qkv._b, K, qkv.out_features))
        op = att.o_proj
        out.append(("o", "", op.quantized_weight, op.scales, op.biases_quant, op.local_in_features,
                    op.out_features))
        out.append(("gate_up", "norm+swiglu", gu._wq, gu._s, gu._b, K, gu.out_features))
        dp = mlp.down_proj
        out.append(("down", "", dp.quantized_weight, dp.scales, dp.biases_quant, dp.local_in_features,
                    dp.out_features))
    lm = model.lm_head
    out.append(("lm_head", "norm", lm.quantized_weight, lm.scales, lm.biases_quant, model.hidden_size,
                lm.local_out_features))
    return out


def qmm_bytes(M, N, K, bits):
    """Algorithmic bytes of one quantized product: weights + bf16 scales/biases + x + y
    (y counted at N columns; the gated gate|up product writes N / 2)."""
    return N * K * bits // 8 + N * (K // 64) * 2 * 2 + M * K * 2 + M * N * 2


def _gemv_io(launches, batch):
    import torch
    dev = torch.device("cuda", 0)
    Ks = {l[5] for l in launches}
    io = {"x": {K: torch.randn((batch, K), device=dev).to(torch.bfloat16) for K in Ks},
          "res": {K: torch.randn((batch, K), device=dev).to(torch.bfloat16) for K in Ks},
          "h": {K: torch.empty((batch, K), dtype=torch.bfloat16, device=dev) for K in Ks},
          "xn": {K: torch.empty((batch, K), dtype=torch.bfloat16, device=dev) for K in Ks},
          "nw": {K: torch.ones(K, dtype=torch.bfloat16, device=dev) for K in Ks},
          "gu": {K: torch.randn((batch, 2 * K), device=dev).to(torch.bfloat16) for K in Ks},
          "y": {N: torch.empty((batch, N), dtype=torch.bfloat16, device=dev) for N in {l[6] for l in launches}},
          "act": {N // 2: torch.empty((batch, N // 2), dtype=torch.bfloat16, device=dev)
                  for N in {l[6] for l in launches}}}
    return io


def _launch_all(launches, io, bits):
    from shardcompute_amd import _lib
    for name, pro, wq, s, b, K, N in launches:
        if pro == "norm+swiglu":
            _lib.qmm_swiglu(io["x"][K], wq, s, b, norm_weight=io["nw"][K], eps=1e-5, residual=io["res"][K],
                            h_out=io["h"][K], xn_out=io["xn"][K], bits=bits, act_out=io["act"][N // 2],
                            gate_up_scratch=io["y"][N])
        elif pro == "norm":
            _lib.qmm_rmsnorm(io["x"][K], io["nw"][K], 1e-5, wq, s, b, residual=io["res"][K], h_out=io["h"][K],
                             xn_out=io["xn"][K], bits=bits, out=io["y"][N])
        else:
            _lib.qmm(io["x"][K], wq, s, b, bits=bits, out=io["y"][N])


def time_gemv_launches(model, batch, bits, reps):
    """Average duration of the decode step's quantized-product launches.

    The launches of one step (every layer's q|k|v, o, gate|up, down and the
    lm_head, on the model's own weights: 4.2 GB, far beyond the 256 MB
    last-level cache) are captured in a HIP graph, which runs them back to back
    with no host gaps; HIP events on the replay stream bracket ``reps`` replays.
    The same is done per projection kind for the per-shape breakdown."""
    import torch
    launches = gemv_launches(model)
    io = _gemv_io(launches, batch)

    def graph_of(ls):
        _launch_all(ls, io, bits)          # warm (kernel attributes set outside capture)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            _launch_all(ls, io, bits)
        return g

    def timed(g, n_launch):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * n_launch)

    avg_us = timed(graph_of(launches), len(launches))
    tot_bytes = sum(qmm_bytes(batch, l[6], l[5], bits) for l in launches)
    per = {}
    for kind in ("qkv", "o", "gate_up", "down", "lm_head"):
        ls = [l for l in launches if l[0] == kind]
        us = timed(graph_of(ls), len(ls))
        nb = qmm_bytes(batch, ls[0][6], ls[0][5], bits)
        per[kind] = {"K": ls[0][5], "N": ls[0][6], "prologue": ls[0][1] or "none", "avg_us": round(us, 3),
                     "GBs": round(nb / (us * 1e-6) / 1e9, 1)}
    bpl = tot_bytes / len(launches)
    log(f"gemv: {len(launches)} launches/step, avg {avg_us:.3f} us, {bpl / 1e6:.2f} MB/launch, "
        f"{bpl / (avg_us * 1e-6) / 1e9:.0f} GB/s")
    return dict(avg_us=avg_us, bytes_per_launch=bpl, GBs=bpl / (avg_us * 1e-6) / 1e9,
                launches_per_step=len(launches), per_shape=per)


def time_prefill_gemms(model, M, bits, reps):
    """Prefill quantized GEMM (kernel B) per projection shape of layer 0 at M rows:
    HIP events on the current stream around ``reps`` back-to-back launches (after a
    warm-up), 2 * M * N * K flops per launch against the 2.5 PFLOP/s dense bf16 peak."""
    import torch
    from shardcompute_amd import _lib
    layer = model.layers[0]
    att, mlp = layer.attention, layer.mlp
    K = model.hidden_size
    shapes = [("qkv", att.qkv._wq, att.qkv._s, att.qkv._b, K, att.qkv.out_features),
              ("o", att.o_proj.quantized_weight, att.o_proj.scales, att.o_proj.biases_quant,
               att.o_proj.local_in_features, att.o_proj.out_features),
              ("gate_up", mlp.gate_up._wq, mlp.gate_up._s, mlp.gate_up._b, K, mlp.gate_up.out_features),
              ("down", mlp.down_proj.quantized_weight, mlp.down_proj.scales, mlp.down_proj.biases_quant,
               mlp.down_proj.local_in_features, mlp.down_proj.out_features)]
    out, tot_fl, tot_us = {}, 0.0, 0.0
    for name, wq, s, b, k, n in shapes:
        x = torch.randn((M, k), device="cuda").to(torch.bfloat16)
        y = torch.empty((M, n), dtype=torch.bfloat16, device="cuda")
        for _ in range(2):
            _lib.qmm(x, wq, s, b, bits=bits, path=_lib.PATH_GEMM, out=y)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            _lib.qmm(x, wq, s, b, bits=bits, path=_lib.PATH_GEMM, out=y)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        fl = 2.0 * M * n * k
        tot_fl += fl * len(model.layers)
        tot_us += us * len(model.layers)
        # context: a dense bf16 GEMM of the same shape (torch.matmul -> hipBLASLt),
        # without the dequantization, on the same inputs
        wd = torch.randn((n, k), device="cuda").to(torch.bfloat16)
        for _ in range(2):
            torch.matmul(x, wd.t())
        e0.record()
        for _ in range(reps):
            torch.matmul(x, wd.t())
        e1.record()
        torch.cuda.synchronize()
        us_d = e0.elapsed_time(e1) * 1e3 / reps
        out[name] = {"K": k, "N": n, "avg_us": round(us, 1), "TFLOPs": round(fl / (us * 1e-6) / 1e12, 1),
                     "frac": round(fl / (us * 1e-6) / MFMA_BF16_PEAK, 4),
                     "dense_bf16_hipblaslt_TFLOPs": round(fl / (us_d * 1e-6) / 1e12, 1)}
        del x, y, wd
    agg = tot_fl / (tot_us * 1e-6)
    log(f"prefill qGEMM at M={M}: " + ", ".join(f"{k} {v['TFLOPs']} TF/s" for k, v in out.items()))
    return {"kernel": f"qgemm_mfma_kernel<{bits}, *>", "M": M, "bound": "mfma", "unit": "TFLOP/s",
            "achieved": round(agg / 1e12, 1), "peak": MFMA_BF16_PEAK / 1e12, "frac": round(agg / MFMA_BF16_PEAK, 4),
            "per_shape": out}


def trunk_bytes(model, cache_len, bits):
    """Algorithmic bytes of one whole-trunk decode launch at batch 1 with ``cache_len``
    positions cached: every layer's q|k|v, o, gate|up and down packed weights + bf16
    scales and biases, the keys and values of cache_len + 1 positions read, the new
    key and value written, the embedding row read and the output row written."""
    att, mlp = model.layers[0].attention, model.layers[0].mlp
    H, I = model.hidden_size, mlp.local_intermediate
    D, Hkv = att.head_dim, att.local_num_kv_heads
    qkvN = (att.local_num_heads + 2 * Hkv) * D
    w = sum(N * K * bits // 8 + N * (K // 64) * 4
            for N, K in ((qkvN, H), (H, att.local_num_heads * D), (2 * I, H), (H, I)))
    kv = 2 * Hkv * (cache_len + 1) * D * 2 + 2 * Hkv * D * 2
    return len(model.layers) * (w + kv) + 2 * H * 2


def time_trunk_launches(dec, reps):
    """Average duration of the whole-trunk launch: HIP events on the launch stream
    around ``reps`` back-to-back eager launches of the plan (each recomputes the same
    step: the cache slot and token id come from the counters it does not advance)."""
    import torch
    plan = dec.bufs.plan
    plan.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        plan.run()
    e1.record()
    torch.cuda.synchronize()
    if plan.status() != 0:
        raise RuntimeError(f"trunk launch gave up (status {plan.status()})")
    return e0.elapsed_time(e1) * 1e3 / reps


def eager_gemv_passes(model, batch, bits, passes):
    """The same launches, eager (for hardware-counter runs, one dispatch at a time)."""
    import torch
    launches = gemv_launches(model)
    io = _gemv_io(launches, batch)
    for _ in range(passes):
        _launch_all(launches, io, bits)
    torch.cuda.synchronize()
    return launches


# ---------------------------------------------------------------- CPU baseline


def host_cpu():
    """Cores this process may run on and the CPU model name (from /proc/cpuinfo)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"affinity_cores": n, "model": model}



def cpu_baseline(model, batch, bits, seconds):
    """The C restatement on decoder layer 0's projections + 1/32 of the lm_head rows."""
    import numpy as np
    import torch
    from oracle import cref

    def u32(t):
        return t.cpu().view(torch.int32).numpy().view(np.uint32)

    def u16(t):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)

    if not cref.available():
        cref.build()
    threads = cref.default_threads()
    launches = gemv_launches(model)
    layer0 = launches[:4]
    name, _, lwq, ls, lb, K, N = launches[-1]
    rows = N // 32
    sample = [(u32(l[2]), u16(l[3]), u16(l[4]), l[5]) for l in layer0]
    lm = (u32(lwq[:rows]), u16(ls[:rows]), u16(lb[:rows]), K)
    rng = np.random.default_rng(0)
    xs = {k: (rng.standard_normal((batch, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
          for k in {s[3] for s in sample}}
    for wq, s, b, k in sample:                   # warm (thread pool, pages)
        cref.qmm_fast_bf16(xs[k], wq, s, b, bits=bits, threads=threads)
    reps, t_layer, t_lm = 0, 0.0, 0.0
    t_start = time.perf_counter()
    while reps == 0 or (time.perf_counter() - t_start) < seconds:
        t0 = time.perf_counter()
        for wq, s, b, k in sample:
            cref.qmm_fast_bf16(xs[k], wq, s, b, bits=bits, threads=threads)
        t1 = time.perf_counter()
        cref.qmm_fast_bf16(xs[lm[3]], lm[0], lm[1], lm[2], bits=bits, threads=threads)
        t2 = time.perf_counter()
        t_layer += t1 - t0
        t_lm += t2 - t1
        reps += 1
    per_token = model.num_layers * t_layer / reps + 32 * t_lm / reps
    host = host_cpu()
    return {"value": round(batch / per_token, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "host_cores": host["affinity_cores"], "cpu_model": host["model"],
            "threads_note": (f"OpenMP threads = min(affinity cores, 16): {threads} of the "
                             f"{host['affinity_cores']} cores this process may run on"),
            "sample": (f"CPU restatement, not MLX (oracle/qmm_fast.c: fp32 accumulation, AVX2 + FMA, OpenMP) of "
                       f"the W{bits} g64 quantized matmuls: "
                       f"decoder layer 0's q|k|v, o, gate|up, down plus lm_head rows [0, {rows}) at M={batch}, "
                       f"{reps} repetitions in {time.perf_counter() - t_start:.1f} s, scaled x{model.num_layers} "
                       f"layers and x32 lm_head rows; attention and norms not included")}



# ---------------------------------------------------------------- further workloads
#
# The other configurations of the measured hot path, each reported beside the
# headline (never required: a failure is logged and reported as an error string).


def _events_us(fn, reps, warm=2):
    """Average duration of fn() over ``reps`` back-to-back calls: HIP events on the
    current stream (the stream the library launches on)."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def zipf_ids(n_vocab, shape, s=1.1, seed=0):
    """Token ids from the bounded Zipf law p(k) ~ k^-s, k = 1..n_vocab, id = k - 1."""
    import numpy as np
    rng = np.random.default_rng(seed)
    p = np.arange(1, n_vocab + 1, dtype=np.float64) ** -s
    p /= p.sum()
    return rng.choice(n_vocab, size=shape, p=p).astype(np.int64)


def bench_vocab_gather(reps=20):
    """Rank 0 of a world_size-2 vocab split of a 128256 x 4096 bf16 table (rows
    [0, 64128)), ids [64, 2048] Zipf(1.1) over the whole vocabulary: the masked
    gather, GB/s on the algorithmic bytes ids + written rows + unique in-shard
    rows read."""
    import numpy as np
    import torch
    from shardcompute_amd import _lib
    V, VL, D = 128256, 64128, 4096
    ids_np = zipf_ids(V, (64, 2048))
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    table = torch.randn((VL, D), generator=g, device="cuda").mul_(0.02).to(torch.bfloat16)
    ids = torch.from_numpy(ids_np).cuda()
    out = torch.empty((64, 2048, D), dtype=torch.bfloat16, device="cuda")
    us = _events_us(lambda: _lib.vocab_gather(ids, table, 0, out=out), reps)
    T = ids_np.size
    inshard = ids_np[ids_np < VL]
    U = int(np.unique(inshard).size)
    nbytes = T * 8 + T * D * 2 + U * D * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {"kernel": "vocab_gather_kernel", "ids": [64, 2048], "table": [VL, D], "vocab": V,
           "in_shard_frac": round(inshard.size / T, 4), "unique_in_shard_rows": U, "bytes": int(nbytes),
           "avg_us": round(us, 2), "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    log(f"vocab gather (config 3): {us:.1f} us, {gbs:.0f} GB/s, U={U}")
    del table, ids, out
    return res


def bench_lm_head_m64(reps=10):
    """The config-3 quantized lm_head: W4 g64 [64128, 4096] on hidden [64, 4096]."""
    import torch
    from shardcompute_amd import _lib
    N, K, M = 64128, 4096, 64
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    wq, s, b = _lib.quantize(torch.randn((N, K), generator=g, device="cuda").mul_(0.02), bits=4)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    us = _events_us(lambda: _lib.qmm(x, wq, s, b, bits=4, out=y), reps)
    nbytes = qmm_bytes(M, N, K, 4)
    gbs = nbytes / (us * 1e-6) / 1e9
    tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
    log(f"lm_head M=64 (config 3): {us:.1f} us, {gbs:.0f} GB/s, {tf:.0f} TFLOP/s")
    del wq, s, b, x, y
    return {"M": M, "N": N, "K": K, "bits": 4, "bytes": int(nbytes), "avg_us": round(us, 2), "GBs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "TFLOPs": round(tf, 1)}


def qmm_kernel_label(M, N, K, cus=256):
    """The kernel sc_qmm_bf16's automatic path takes for an M x K -> N product (the
    choice csrc/abi.hip and csrc/qgemm.hip make, restated for the sweep's labels)."""
    band = K % 512 == 0 and (M <= 160 if M > 32 else K >= 4096 if M == 8 else
                             M > 8 and (K > 4096 or N <= 8192))
    if band:
        return "band"
    if M <= 32:
        return "gemv"
    tiles256 = ((M + 255) // 256) * ((N + 255) // 256)
    return "gemm, K split" if 4 * tiles256 <= cus and K // 64 >= 64 else "gemm"


SWEEP_KN = [(2048, 2560), (2048, 5632), (5632, 2048), (4096, 6144), (4096, 14336), (14336, 4096)]
SWEEP_M = [1, 8, 32, 512, 2048]


def bench_qmm_sweep(reps=5):
    """The standalone quantized-linear sweep: x bf16 N(0,1) [M, K], W [N, K] N(0, 0.02)
    quantized W4 and W8 g64, every (K, N) of the TinyLlama and Llama-3-8B projections at
    M in {1, 8, 32, 512, 2048}, through sc_qmm_bf16 (the kernel it selects).

    GPU: enough copies of the packed weights to exceed the 256 MB last-level cache
    (at least 512 MB in all), one product per copy captured in a HIP graph, HIP events
    around ``reps`` replays; GB/s on the algorithmic bytes (M <= 32) or TFLOP/s
    (M >= 512) against 8 TB/s and 2.5 PFLOP/s.  CPU: the vectorised C restatement
    (fp32 accumulation, AVX2 + FMA, OpenMP on this host's cores; not MLX) on a sample
    of the same product (min(M, 64) rows of x, min(N, 256) weight rows), scaled
    linearly to the full M x N."""
    import numpy as np
    import torch
    from oracle import cref
    from shardcompute_amd import _lib
    if not cref.available():
        cref.build()
    threads = cref.default_threads()
    host = host_cpu()
    rows = []
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    for bits in (4, 8):
        for K, N in SWEEP_KN:
            wq, sc, bi = _lib.quantize(torch.randn((N, K), generator=g, device="cuda").mul_(0.02), bits=bits)
            wbytes = N * K * bits // 8 + N * (K // 64) * 4
            copies = max(1, min(200, -(-(512 << 20) // wbytes)))
            ws = [(wq, sc, bi)] + [(wq.clone(), sc.clone(), bi.clone()) for _ in range(copies - 1)]
            wq_h = wq[:256].cpu().view(torch.int32).numpy().view(np.uint32)
            s_h = sc[:256].cpu().view(torch.int16).numpy().view(np.uint16)
            b_h = bi[:256].cpu().view(torch.int16).numpy().view(np.uint16)
            for M in SWEEP_M:
                x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
                y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
                for w in ws[:2]:
                    _lib.qmm(x, *w, bits=bits, out=y)          # warm: plans and scratch outside capture
                torch.cuda.synchronize()
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for w in ws:
                        _lib.qmm(x, *w, bits=bits, out=y)
                gr.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    gr.replay()
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
                nbytes = qmm_bytes(M, N, K, bits)
                flops = 2.0 * M * N * K
                kernel = qmm_kernel_label(M, N, K)
                row = {"bits": bits, "M": M, "K": K, "N": N, "kernel": kernel, "gpu_us": round(us, 2)}
                if M <= 32:
                    gbs = nbytes / (us * 1e-6) / 1e9
                    row.update(bound="hbm", GBs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
                else:
                    tf = flops / (us * 1e-6) / 1e12
                    row.update(bound="mfma", TFLOPs=round(tf, 1), frac=round(tf * 1e12 / MFMA_BF16_PEAK, 4))
                # CPU restatement on a sample, scaled to the full product
                Ms, Ns = min(M, 64), min(N, 256)
                x_h = x[:Ms].cpu().view(torch.int16).numpy().view(np.uint16)
                cref.qmm_fast_bf16(x_h, wq_h[:Ns], s_h[:Ns], b_h[:Ns], bits=bits, threads=threads)
                t0 = time.perf_counter()
                n_cpu = 0
                while n_cpu == 0 or time.perf_counter() - t0 < 0.05:
                    cref.qmm_fast_bf16(x_h, wq_h[:Ns], s_h[:Ns], b_h[:Ns], bits=bits, threads=threads)
                    n_cpu += 1
                cpu_us = (time.perf_counter() - t0) / n_cpu * 1e6 * (M / Ms) * (N / Ns)
                row.update(cpu_us_est=round(cpu_us, 1), gpu_vs_cpu=round(cpu_us / us, 1))
                rows.append(row)
                del x, y, gr
            del ws, wq, sc, bi
            torch.cuda.empty_cache()
    for r in rows:
        perf = f"{r['GBs']:.0f} GB/s" if r["bound"] == "hbm" else f"{r['TFLOPs']:.0f} TFLOP/s"
        log(f"sweep W{r['bits']} M={r['M']:4d} K={r['K']:5d} N={r['N']:5d} {r['kernel']:4s}: {r['gpu_us']:8.2f} us "
            f"{perf:>14s} ({100 * r['frac']:.1f} %), CPU {r['cpu_us_est'] / 1e3:.2f} ms (x{r['gpu_vs_cpu']})")
    return {"rows": rows,
            "cpu": {"kind": "CPU restatement, not MLX: oracle/qmm_fast.c (fp32 accumulation, AVX2 + FMA, OpenMP)",
                    "threads": threads, "host_cores": host["affinity_cores"], "cpu_model": host["model"],
                    "sample": "min(M, 64) rows of x and min(N, 256) weight rows, repeated for >= 50 ms, "
                              "scaled linearly by (M / rows) x (N / weight rows)"},
            "gpu": "graph replays over >= 512 MB of weight copies; GB/s at M <= 32, TFLOP/s at M >= 512"}


def bench_w8_gemv(reps):
    """Batch-1 decode qGEMV at 8 bits on the Llama-3-8B projection shapes (4 layers'
    distinct weights + the lm_head, more than the 256 MB last-level cache)."""
    import torch
    model = build_model(LLAMA3_8B, 4, 8, 64, seed=5)
    g = time_gemv_launches(model, 1, 8, reps)
    del model
    torch.cuda.empty_cache()
    return {"kernel": "qgemv_m1_kernel<8, *, *>", "avg_launch_us": round(g["avg_us"], 3),
            "bytes_per_launch": round(g["bytes_per_launch"]), "GBs": round(g["GBs"], 1),
            "frac": round(g["GBs"] / HBM_PEAK_GBS, 4), "per_shape": g["per_shape"]}


def time_prefill_attention(cfg, B, P, reps):
    """The prefill attention of one layer (B x P new positions, empty cache before
    them) on random q, k, v: average launch time and TFLOP/s of the causal half."""
    import math
    import torch
    from shardcompute_amd import _lib
    H, Hkv, D = cfg["heads"], cfg["kv_heads"], cfg["hidden"] // cfg["heads"]
    T_cap = (P + 31) // 32 * 32
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    q = torch.randn((B * P, H * D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn((B, Hkv, T_cap, D), generator=g, device="cuda").to(torch.bfloat16)
    vt = torch.randn((B, Hkv, D, T_cap), generator=g, device="cuda").to(torch.bfloat16)
    cnt = torch.zeros(2, dtype=torch.int32, device="cuda")
    out = torch.empty((B * P, H * D), dtype=torch.bfloat16, device="cuda")
    scale = 1.0 / math.sqrt(D)
    _lib.attention(q, B, P, H, Hkv, D, kc, vt, cnt, scale, out=out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        _lib.attention(q, B, P, H, Hkv, D, kc, vt, cnt, scale, out=out)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    flops = 4.0 * B * H * D * P * (P + 1) / 2
    log(f"attn-only: {B} x {P} positions, {H} q / {Hkv} kv heads of {D}: {us:.1f} us per launch, "
        f"{flops / us / 1e6:.0f} TFLOP/s (causal half), {reps} launches")


def time_batched_gemv(reps):
    """W4 quantized products of the batched decode steps on random weights: per shape,
    the average time of one call (the 9-32-row GEMV plus its split-K pass) over
    `reps` back-to-back calls, and GB/s of its algorithmic bytes (packed weights,
    scales and biases, x and y).  A 256 MiB copy runs first (counter scale)."""
    import torch
    from shardcompute_amd import _lib
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    shapes = [("70B-shard q|k|v", 32, 8192, 1280), ("70B-shard o", 32, 1024, 8192),
              ("70B-shard gate|up", 32, 8192, 7168), ("70B-shard down", 32, 3584, 8192),
              ("8B q|k|v", 16, 4096, 6144), ("8B o", 16, 4096, 4096),
              ("8B gate|up", 16, 4096, 28672), ("8B down", 16, 14336, 4096)]
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    for name, M, K, N in shapes:
        wq, s, b = _lib.quantize(torch.randn((N, K), generator=g, device="cuda").mul_(0.02), bits=4)
        x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        _lib.qmm(x, wq, s, b, bits=4, out=y)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            _lib.qmm(x, wq, s, b, bits=4, out=y)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = N * K // 2 + N * (K // 64) * 4 + M * K * 2 + M * N * 2
        log(f"gemv16-only: {name} M={M} K={K} N={N}: {us:.2f} us per call, {nbytes / us / 1e3:.0f} GB/s "
            f"({nbytes / 1e6:.2f} MB), {reps} calls")
        del wq, s, b, x, y


def timed_prefill(model, ids, cache):
    """Seconds of the prefill forward of ``ids`` into ``cache`` (last position's
    logits), after one untimed prefill of the same shape into a scratch cache (the
    first launch of each kernel loads its code object)."""
    import torch
    B, P = ids.shape
    scratch = model.new_cache(B, cache.capacity)
    asyncio.run(model.forward(ids, past_key_values=scratch, use_cache=True, last_only=True))
    del scratch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits, _ = asyncio.run(model.forward(ids, past_key_values=cache, use_cache=True, last_only=True))
    torch.cuda.synchronize()
    return time.perf_counter() - t0, logits


def decode_run(model, B, prompt, steps, warm=8, seed=1):
    """Prefill B random prompts of ``prompt`` tokens, then greedy decode: returns
    (prefill seconds, decode tokens/s over ``steps`` timed steps, ms per step,
    whether the whole-trunk plan ran)."""
    import torch
    from shardcompute_amd import _lib
    from shardcompute_amd.executor import DecodeGraph
    cap = prompt + warm + steps + 8
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    ids = torch.randint(0, model.vocab_size, (B, prompt), generator=gen, device="cuda", dtype=torch.int64)
    cache = model.new_cache(B, cap)
    pre_s, logits = timed_prefill(model, ids, cache)
    tokens = torch.zeros((B, warm + steps + 2), dtype=torch.int32, device="cuda")
    dec = DecodeGraph(model, cache, tokens)
    _lib.argmax(logits.reshape(B, -1), ids=dec.bufs.ids.view(-1), tokens=tokens, step=cache.counters[1:])
    _lib.add_i32(cache.counters[1:], 1, n=1)
    dec.run(1)
    dec.run(warm)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.run(steps)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    trunk = dec.bufs.plan is not None
    if trunk and dec.bufs.plan.status() != 0:
        raise RuntimeError("whole-trunk launch gave up waiting")
    del dec, cache, tokens, logits
    return pre_s, B * steps / el, el / steps * 1e3, trunk


def bench_decode_config(name, cfg, bits, B, prompt, steps, layers=None, world_size=1):
    import torch
    L = layers or cfg["layers"]
    t0 = time.perf_counter()
    model = build_model(cfg, L, bits, prompt + steps + 32, seed=7, world_size=world_size)
    build_s = time.perf_counter() - t0
    pre_s, tok_s, ms, trunk = decode_run(model, B, prompt, steps)
    log(f"{name}: built in {build_s:.1f} s, prefill {B}x{prompt} in {pre_s * 1e3:.0f} ms, decode {tok_s:.1f} tok/s "
        f"({ms:.3f} ms/step, {'whole-trunk' if trunk else 'per-op'} path)")
    res = {"layers": L, "bits": bits, "batch": B, "prefill_tokens": prompt, "steps": steps,
           "world_size": world_size, "rank": 0, "tok_s": round(tok_s, 1), "ms_per_step": round(ms, 4),
           "prefill_ms": round(pre_s * 1e3, 1), "path": "whole-trunk launch" if trunk else "per-op launches"}
    del model
    torch.cuda.empty_cache()
    return res


def bench_batch16(model, steps):
    """Batch-16 greedy decode of the headline model after a 2048-token prefill per sequence."""
    pre_s, tok_s, ms, trunk = decode_run(model, 16, 2048, steps)
    log(f"8B batch 16: prefill 16x2048 in {pre_s * 1e3:.0f} ms, decode {tok_s:.1f} tok/s ({ms:.3f} ms/step)")
    return {"batch": 16, "prefill_tokens": 2048, "steps": steps, "tok_s": round(tok_s, 1),
            "ms_per_step": round(ms, 4), "prefill_ms": round(pre_s * 1e3, 1), "path": "per-op launches"}


def run_extras(model, args):
    import torch
    out = {}
    jobs = [
        ("vocab_gather_config3", lambda: bench_vocab_gather()),
        ("lm_head_m64_config3", lambda: bench_lm_head_m64()),
        ("batch16_llama3_8b_w4", lambda: bench_batch16(model, 32)),
        ("qmm_sweep_config2", lambda: bench_qmm_sweep()),
    ]
    if args.extras_models:
        jobs += [
            ("w8_decode_gemv_llama3_8b", lambda: bench_w8_gemv(args.kernel_reps)),
            ("tinyllama_w4_bs1", lambda: bench_decode_config("TinyLlama W4 bs1", TINYLLAMA, 4, 1, 32, 128)),
            ("llama3_70b_rank0_of_8_w4_bs32", lambda: bench_decode_config(
                "70B rank-0 shard W4 bs32", LLAMA3_70B, 4, 32, 1024, 32, world_size=8)),
            ("llama3_70b_rank0_of_8_w8_bs32", lambda: bench_decode_config(
                "70B rank-0 shard W8 bs32", LLAMA3_70B, 8, 32, 1024, 32, world_size=8)),
        ]
    for name, fn in jobs:
        try:
            out[name] = fn()
        except Exception as e:           # reported, never required
            log(f"{name}: failed: {e!r}")
            out[name] = {"error": repr(e)[:300]}
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out

# ---------------------------------------------------------------- main


def main():
    args = parse_args()
    if args.gpus != 1:
        log(f"bench.py measures one GPU: --gpus {args.gpus} is not supported by this build "
            f"(no collectives; the multi-GPU sharding is a design note only)")
        sys.exit(2)
    import torch
    from shardcompute_amd import _lib
    from shardcompute_amd.executor import DecodeGraph
    if not torch.cuda.is_available():
        log("no GPU visible")
        sys.exit(1)
    _lib.load()
    cfg = dict(LLAMA3_8B if args.model == "llama3-8b" else TINYLLAMA)
    if args.layers is None:
        args.layers = cfg["layers"]
    B, P, K, W = args.batch, args.prefill, args.steps, args.warmup
    if args.attn_only:
        time_prefill_attention(cfg, B, P, args.kernel_reps)
        return
    if args.gemv16_only:
        time_batched_gemv(args.kernel_reps)
        return
    if args.sweep_only:
        print(json.dumps(bench_qmm_sweep()), flush=True)
        return
    if args.batched_decode_only:
        out = {"batch16_llama3_8b_w4": bench_decode_config("Llama-3-8B W4 bs16", LLAMA3_8B, 4, 16, 2048, K),
               "llama3_70b_rank0_of_8_w4_bs32": bench_decode_config("70B rank-0 shard W4 bs32", LLAMA3_70B, 4, 32,
                                                                    1024, K, world_size=8)}
        print(json.dumps(out), flush=True)
        return
    if args.shard_head_only:
        print(json.dumps({"vocab_gather_config3": bench_vocab_gather(),
                          "lm_head_m64_config3": bench_lm_head_m64(args.kernel_reps)}), flush=True)
        return
    capacity = P + W + K + 8
    t_build = time.perf_counter()
    model = build_model(cfg, args.layers, args.bits, capacity)
    log(f"built {args.layers}-layer W{args.bits} model in {time.perf_counter() - t_build:.1f} s "
        f"({torch.cuda.memory_allocated() / 2**30:.2f} GiB allocated)")

    if args.kernels_only:
        # a plain copy of known size first (256 MiB read + 256 MiB written), to scale
        # the HBM counters, then the decode step's quantized products, eager
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        ls = eager_gemv_passes(model, B, args.bits, args.kernel_reps)
        log(f"kernels-only: 3 copies of {src.numel()} bytes, {args.kernel_reps} x {len(ls)} quantized products")
        return

    if args.gemm_only:
        gemm = time_prefill_gemms(model, P * B, args.bits, args.kernel_reps)
        log(f"gemm-only: {args.kernel_reps} launches per shape at M = {P * B}, "
            f"{gemm['achieved']} TFLOP/s over the four shapes")
        return

    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    ids = torch.randint(0, cfg["vocab"], (B, P), generator=gen, device="cuda", dtype=torch.int64)
    cache = model.new_cache(B, capacity)
    prefill_s, logits = timed_prefill(model, ids, cache)
    log(f"prefill {P} tokens x {B}: {prefill_s * 1e3:.1f} ms (after one untimed prefill)")

    tokens = torch.zeros((B, W + K + 2), dtype=torch.int32, device="cuda")
    dec = DecodeGraph(model, cache, tokens)
    if args.trunk_timeline:
        if dec.bufs.plan is None:
            log("trunk-timeline: the whole-trunk plan does not apply to this configuration")
            sys.exit(2)
        _lib.argmax(logits.reshape(B, -1), ids=dec.bufs.ids.view(-1), tokens=tokens, step=cache.counters[1:])
        _lib.add_i32(cache.counters[1:], 1, n=1)
        dec.run(1 + W)                  # eager step, capture, warm graph replays
        plan = dec.bufs.plan
        plan.trace(True)
        t_us = time_trunk_launches(dec, args.kernel_reps)
        tl = plan.timeline()
        plan.trace(False)
        shape = "Llama-3-8B" if args.model == "llama3-8b" else "TinyLlama-1.1B"
        tl.update({"workload": f"{shape}-shape W{args.bits}g64 whole-trunk decode launch, batch 1, context "
                               f"{cache.length}", "layers": args.layers, "avg_launch_us": round(t_us, 1),
                   "stamps": "s_memrealtime (100 MHz) by each workgroup's control wave, last of "
                             f"{args.kernel_reps + 1} back-to-back launches"})
        print(json.dumps(tl), flush=True)
        return
    if args.trunk_only:
        if dec.bufs.plan is None:
            log("trunk-only: the whole-trunk plan does not apply to this configuration")
            sys.exit(2)
        # a plain copy of known size first (256 MiB read + 256 MiB written), to scale
        # the HBM counters, then eager trunk launches
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        us = time_trunk_launches(dec, args.kernel_reps)
        log(f"trunk-only: 3 copies of {src.numel()} bytes, {args.kernel_reps + 1} trunk launches, "
            f"{us:.1f} us each, {trunk_bytes(model, cache.length, args.bits)} bytes algorithmic per launch")
        return
    _lib.argmax(logits.reshape(B, -1), ids=dec.bufs.ids.view(-1), tokens=tokens, step=cache.counters[1:])
    _lib.add_i32(cache.counters[1:], 1, n=1)
    dec.run(1)            # eager step, then capture
    dec.run(W)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.run(K)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    tok_s = B * K / el
    ms_step = el / K * 1e3
    log(f"decode: {K} steps in {el * 1e3:.1f} ms -> {ms_step:.3f} ms/step, {tok_s:.1f} tok/s")
    first = tokens[0, :8].tolist()

    trunk = None
    if dec.bufs.plan is not None:
        t_us = time_trunk_launches(dec, args.kernel_reps)
        t_bytes = trunk_bytes(model, cache.length, args.bits)
        trunk = dict(avg_us=t_us, bytes=t_bytes, GBs=t_bytes / (t_us * 1e-6) / 1e9)
        log(f"trunk: {t_us:.1f} us/launch, {t_bytes / 1e9:.3f} GB/launch, {trunk['GBs']:.0f} GB/s")
    g = time_gemv_launches(model, B, args.bits, args.kernel_reps)
    gemm = time_prefill_gemms(model, P * B, args.bits, args.kernel_reps) if P * B >= 128 else None
    step_gemv_bytes = g["bytes_per_launch"] * g["launches_per_step"]
    step_gemv_ms = g["avg_us"] * g["launches_per_step"] / 1e3
    def traffic_of(path):
        if os.path.exists(path):
            with open(path) as f:
                return json.load(f).get("hbm_bytes_per_launch")
        return None

    qroof = {"bound": "hbm", "achieved": round(g["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
             "frac": round(g["GBs"] / HBM_PEAK_GBS, 4), "traffic": traffic_of(TRAFFIC_FILE),
             "kernel": (f"qgemv_m1_kernel<{args.bits}, *, *>" if B == 1 else f"qgemv_dma_kernel<{args.bits}, 8, *, *>")
                       if B <= 8 else "qgemv",
             "avg_launch_us": round(g["avg_us"], 3), "bytes_per_launch": round(g["bytes_per_launch"]),
             "launches_per_step": g["launches_per_step"]}
    if trunk is not None:
        hd = cfg["hidden"] // cfg["heads"]
        roof = {"bound": "hbm", "achieved": round(trunk["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(trunk["GBs"] / HBM_PEAK_GBS, 4),
                "traffic": traffic_of(TRUNK_TRAFFIC_FILE) if args.bits == 4 and args.layers == 32 else None,
                "kernel": f"decode_step_kernel<{args.bits}, {hd}, {4 if hd == 128 else 8}>",
                "avg_launch_us": round(trunk["avg_us"], 2),
                "bytes_per_launch": int(trunk["bytes"]), "launches_per_step": 1}
    else:
        roof = qroof

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(model, B, args.bits, args.cpu_seconds)
        except Exception as e:       # the baseline is reported, never required
            log(f"cpu baseline unavailable: {e}")

    extras = run_extras(model, args) if args.extras and B == 1 and args.layers == 32 else None

    kv_bytes = 2 * args.layers * B * cfg["kv_heads"] * (cfg["hidden"] // cfg["heads"]) * 2 * (P + W + K // 2)
    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: random-init N(0,0.02) weights quantized W4 g64 on the GPU, "
                                 "uniform random prompt ids",
        "config": {"workload": f"Llama-3-8B-shape W{args.bits}g64 greedy decode, batch {B}, after a {P}-token "
                               f"prefill", "batch": B, "prefill_tokens": P, "layers": args.layers,
                   "hidden": cfg["hidden"], "intermediate": cfg["inter"], "heads": cfg["heads"],
                   "kv_heads": cfg["kv_heads"], "vocab": cfg["vocab"], "weights": f"W{args.bits} g64, bf16 s/b",
                   "activations": "bf16, fp32 accumulate", "decode": "HIP graph replays of 8 steps"},
        "roofline": roof,
        "qgemv_roofline": qroof,
        "cpu_baseline": cpu,
        "prefill": {"tokens": B * P, "ms": round(prefill_s * 1e3, 2), "tok_s": round(B * P / prefill_s, 1),
                    "qgemm_roofline": gemm},
        "decode_step": {"path": "whole-trunk launch + lm_head GEMV with the greedy selection" if trunk is not None
                        else "per-op launches", "gemv_ms": round(step_gemv_ms, 4), "gemv_bytes": int(step_gemv_bytes),
                        "kv_bytes_avg": int(kv_bytes),
                        "step_hbm_frac": round((step_gemv_bytes + kv_bytes) / (ms_step * 1e-3) / 1e9
                                               / HBM_PEAK_GBS, 4)},
        "gemv_per_shape": g["per_shape"],
        "first_tokens": first,
        "other_configs": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
