"""The batch-1 decode trunk as one persistent launch (``sc_decode_plan_*``).

``TrunkPlan`` binds a loaded quantized :class:`ParallelTransformer`, its KV cache
and the step buffers to the library's whole-trunk decode kernel: embedding,
every layer's RMSNorm / q|k|v / RoPE + cache append + attention / o_proj /
RMSNorm / gate|up + SiLU gate / down_proj with the residual adds, for one token
of one sequence (``parallel/transformer.py:537-559`` at S = 1).  After
:meth:`TrunkPlan.run` the step buffer ``h`` holds the residual stream that the
final norm + lm_head read; every layer's cache holds the new position.

The plan reads the token id, the cache slot and the weights through device
pointers captured at construction, so one plan serves every decode step of the
cache it was built for (also inside a captured HIP graph).  It keeps references
to every tensor it points at.  Reloading weights or replacing the cache needs a
new plan.
"""
import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

_p = ctypes.c_void_p


class _Layer(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("wq_qkv", "s_qkv", "b_qkv", "wq_o", "s_o", "b_o", "wq_gu", "s_gu", "b_gu",
                                  "wq_down", "s_down", "b_down", "ln_in", "ln_post", "kc", "vt")]


class _Model(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("hidden", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("num_heads", ctypes.c_int), ("num_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("bits", ctypes.c_int), ("group_size", ctypes.c_int), ("eps", ctypes.c_float),
                ("scale", ctypes.c_float), ("embed", _p), ("vocab_start", ctypes.c_int64),
                ("vocab_local", ctypes.c_int64), ("cos_t", _p), ("sin_t", _p), ("table_len", ctypes.c_int),
                ("pos_offset", ctypes.c_int), ("T_cap", ctypes.c_int), ("counters", _p), ("ids", _p),
                ("h_out", _p)]


def _bias_free(lin) -> bool:
    return not getattr(lin, "has_bias", False) or getattr(lin, "bias", None) is None


def eligible(model, cache) -> Tuple[bool, str]:
    """Whether ``model`` with ``cache`` fits the whole-trunk kernel (else the
    per-op path runs).  Shapes the kernel rejects are found at plan creation."""
    from .parallel.embedding import ParallelEmbedding, VocabParallelEmbedding
    if cache.batch != 1:
        return False, "batch > 1"
    if not model.use_quantized:
        return False, "dense weights"
    from .communicator import IdentityCommunicator
    if model.communicator is not None and not isinstance(model.communicator, IdentityCommunicator):
        return False, "collectives"
    emb = model.embed_tokens
    if isinstance(emb, VocabParallelEmbedding):
        if emb.weight is None:
            return False, "embedding not loaded"
    elif isinstance(emb, ParallelEmbedding):
        if model.world_size != 1 or emb.padding_idx is not None or emb.weight is None:
            return False, "dim-sharded or padded embedding"
    else:
        return False, "quantized embedding"
    for layer in model.layers:
        att, mlp = layer.attention, layer.mlp
        if not att.use_quantized or att.head_dim not in (64, 128):
            return False, "head_dim"
        # the kernels built: up to 4 query heads per kv head at head_dim 128, 8 at 64
        if att.local_num_heads // att.local_num_kv_heads > (4 if att.head_dim == 128 else 8):
            return False, "query heads per kv head"
        if not all(_bias_free(x) for x in (att.q_proj, att.k_proj, att.v_proj, att.o_proj)):
            return False, "attention linear bias"
        if not mlp.fused_swiglu:
            return False, "MLP activation"
        if not (layer.input_layernorm.fusable and layer.post_attention_layernorm.fusable):
            return False, "norm bias"
        if not all(_bias_free(x) for x in (mlp.gate_proj, mlp.up_proj, mlp.down_proj)):
            return False, "MLP linear bias"
        bits = {att.q_proj.bits, att.o_proj.bits, mlp.gate_proj.bits, mlp.down_proj.bits}
        if bits != {model.quantization_bits}:
            return False, "mixed bits"
    return True, ""


class TrunkPlan:
    def __init__(self, model, cache, ids: torch.Tensor, h_out: torch.Tensor, pos_offset: int = 0):
        ok, why = eligible(model, cache)
        if not ok:
            raise ValueError(f"the whole-trunk decode kernel does not apply: {why}")
        lib = _lib.load()
        L = len(model.layers)
        att0, mlp0 = model.layers[0].attention, model.layers[0].mlp
        H, Hk, D = att0.local_num_heads, att0.local_num_kv_heads, att0.head_dim
        hid, I = model.hidden_size, mlp0.local_intermediate
        if ids.dtype != torch.int32 or ids.numel() != 1 or not ids.is_cuda:
            raise ValueError("ids must be one int32 device element")
        if h_out.dtype != torch.bfloat16 or h_out.numel() != hid or not h_out.is_contiguous():
            raise ValueError(f"h_out must be a contiguous bf16 tensor of {hid} elements")
        keep = [ids, h_out, cache.counters]
        layers = (_Layer * L)()
        for i, layer in enumerate(model.layers):
            att, mlp = layer.attention, layer.mlp
            for f in (att.qkv, mlp.gate_up):
                if not f._current():
                    f.build()
            o, d = att.o_proj, mlp.down_proj
            t = {"qkv": (att.qkv._wq, att.qkv._s, att.qkv._b), "o": (o.quantized_weight, o.scales, o.biases_quant),
                 "gu": (mlp.gate_up._wq, mlp.gate_up._s, mlp.gate_up._b),
                 "down": (d.quantized_weight, d.scales, d.biases_quant)}
            for name, (wq, s, b) in t.items():
                for x in (wq, s, b):
                    if not x.is_contiguous():
                        raise ValueError(f"layer {i} {name}: weights must be contiguous")
                setattr(layers[i], f"wq_{name}", wq.data_ptr())
                setattr(layers[i], f"s_{name}", s.data_ptr())
                setattr(layers[i], f"b_{name}", b.data_ptr())
                keep += [wq, s, b]
            layer.input_layernorm._check()
            layer.post_attention_layernorm._check()
            layers[i].ln_in = layer.input_layernorm.weight.data_ptr()
            layers[i].ln_post = layer.post_attention_layernorm.weight.data_ptr()
            keep += [layer.input_layernorm.weight, layer.post_attention_layernorm.weight]
            layers[i].kc = cache.k[i].data_ptr()
            layers[i].vt = cache.vt[i].data_ptr()
        keep += [cache.k, cache.vt]
        emb = model.embed_tokens
        table = emb.weight
        cos_t, sin_t = att0.rope.tables(cache.capacity + pos_offset, table.device)
        keep += [table, cos_t, sin_t]
        m = _Model()
        m.num_layers, m.hidden, m.intermediate = L, hid, I
        m.num_heads, m.num_kv_heads, m.head_dim = H, Hk, D
        m.bits, m.group_size = model.quantization_bits, model.quantization_group_size
        m.eps = float(model.layers[0].input_layernorm.eps)
        m.scale = float(att0.scale)
        m.embed = table.data_ptr()
        m.vocab_start = int(getattr(emb, "vocab_start", 0))
        m.vocab_local = int(table.shape[0])
        m.cos_t, m.sin_t = cos_t.data_ptr(), sin_t.data_ptr()
        m.table_len = int(cos_t.shape[0])
        m.pos_offset = int(pos_offset)
        m.T_cap = int(cache.capacity)
        m.counters = cache.counters.data_ptr()
        m.ids = ids.data_ptr()
        m.h_out = h_out.data_ptr()
        handle = ctypes.c_void_p()
        with torch.cuda.device(table.device):
            rc = lib.sc_decode_plan_create(ctypes.byref(m), layers, ctypes.byref(handle))
        _lib._check(rc, "sc_decode_plan_create")
        self._handle = handle
        self._keep = keep
        self.device = table.device
        self.h_out = h_out

    def run(self):
        """Enqueue one decode step of the trunk on the current stream."""
        lib = _lib.load()
        rc = lib.sc_decode_plan_run(self._handle, _lib._stream(self.h_out))
        _lib._check(rc, "sc_decode_plan_run")
        return self.h_out

    def status(self) -> int:
        """0 when every launch so far completed; nonzero when one gave up (synchronous)."""
        lib = _lib.load()
        v = ctypes.c_uint32(0)
        _lib._check(lib.sc_decode_plan_status(self._handle, ctypes.byref(v)), "sc_decode_plan_status")
        return int(v.value)

    # -------------------------------------------------------------- op timeline

    OP_KINDS = ("qkv", "attn", "merge", "o", "gate_up", "down")

    def trace(self, enable: bool = True):
        """Make later launches record the per-op timeline (allocates a stamp buffer
        once; not under graph capture).  ``trace(False)`` stops recording; the buffer
        lives until the plan is closed, so graphs captured while tracing stay valid."""
        lib = _lib.load()
        _lib._check(lib.sc_decode_plan_trace(self._handle, 1 if enable else 0), "sc_decode_plan_trace")

    def read_trace(self):
        """Stamps of the last launch: int64 [workgroups, ops, 4] in microseconds from
        the earliest stamp (per op: items computed, output published, input polled,
        input staged), synchronously."""
        import numpy as np
        lib = _lib.load()
        P, n = ctypes.c_int(), ctypes.c_int()
        _lib._check(lib.sc_decode_plan_read_trace(self._handle, None, 0, ctypes.byref(P), ctypes.byref(n)),
                    "sc_decode_plan_read_trace")
        buf = np.zeros(P.value * n.value * 4, dtype=np.uint32)
        _lib._check(lib.sc_decode_plan_read_trace(self._handle, ctypes.c_void_p(buf.ctypes.data), buf.size,
                                                  ctypes.byref(P), ctypes.byref(n)), "sc_decode_plan_read_trace")
        t = buf.reshape(P.value, n.value, 4).astype(np.int64)
        t = t - t[t > 0].min()
        return t.astype(np.float64) * 0.01          # 100 MHz clock -> us

    def timeline(self):
        """Per op kind, averaged over the layers away from the ends, in microseconds:
        ``span`` (op staged to the next op staged, on the slowest workgroup),
        ``work`` (median and max over workgroups of staged -> computed), ``straggle``
        (slowest workgroup's publish after the median one's), ``publish`` (computed ->
        published), ``exchange`` (slowest producer's publish -> median consumer's
        input polled) and ``stage`` (polled -> staged) of the op that follows."""
        import numpy as np
        t = self.read_trace()
        comp, pub, pol, stg = t[..., 0], t[..., 1], t[..., 2], t[..., 3]
        nops = t.shape[1]
        L = (nops - 1) // 6
        mid = range(1, L - 1) if L >= 3 else range(L)     # layers away from the ends
        out = {}
        for k, name in enumerate(self.OP_KINDS):
            js = [1 + 6 * l + k for l in mid if 1 + 6 * l + k + 1 < nops]

            def avg(f):
                return float(np.mean([f(j) for j in js]))
            out[name] = {
                "span": avg(lambda j: stg[:, j + 1].max() - stg[:, j].max()),
                "work_median": avg(lambda j: np.median(comp[:, j] - stg[:, j])),
                "work_max": avg(lambda j: (comp[:, j] - stg[:, j]).max()),
                "straggle": avg(lambda j: pub[:, j].max() - np.median(pub[:, j])),
                "publish": avg(lambda j: np.median(pub[:, j] - comp[:, j])),
                "exchange": avg(lambda j: np.median(pol[:, j + 1]) - pub[:, j].max()),
                "stage_next": avg(lambda j: np.median(stg[:, j + 1] - pol[:, j + 1])),
            }
        per_layer = float(np.mean([stg[:, 1 + 6 * (l + 1)].max() - stg[:, 1 + 6 * l].max()
                                   for l in mid if 1 + 6 * (l + 1) < nops]))
        return {"per_layer_us": per_layer, "ops": out}

    def close(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value:
            _lib.load().sc_decode_plan_destroy(h)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def maybe_plan(model, cache, ids, h_out) -> Optional[TrunkPlan]:
    """A TrunkPlan when the model and cache fit the kernel, else None."""
    ok, _ = eligible(model, cache)
    if not ok:
        return None
    try:
        return TrunkPlan(model, cache, ids, h_out)
    except RuntimeError as e:
        if "-2" in str(e):          # unsupported configuration: the per-op path runs
            return None
        raise
