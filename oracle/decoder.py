"""Decoder wiring restated in numpy — TEST INFRASTRUCTURE ONLY.

Follows the reference's per-rank forward at world_size = 1:

* ``rms_norm``       ``parallel/transformer.py:46-61``  (``x / sqrt(mean(x^2) + eps) * w``)
* ``rope_cos_sin`` / ``apply_rope``  ``parallel/attention.py:54-59,66-92,130-151``
  (inverse frequencies ``base^(-2i/d)`` in fp32, rotate-half, positions offset by
  the cache length ``:421-427``)
* ``attention``      ``parallel/attention.py:403-471`` (QKV, RoPE, KV concat,
  GQA repeat, ``q k^T / sqrt(d)``, causal ``triu(k = kv - s + 1)``, softmax, ``@ v``,
  o_proj)
* ``mlp``            ``parallel/mlp.py:238-254`` (gated ``down(f(gate(x)) * up(x))``,
  ungated ``down(f(up(x)))``; the activations f of ``:159-180``: silu/swish,
  gelu = ``x * sigmoid(1.702 x)``, gelu_new (tanh form), relu, gelu_exact (erf))
* ``rms_norm`` with the optional LayerNorm-style bias of ``transformer.py:57-59``
* ``block``          ``parallel/transformer.py:237-254`` (pre-norm residual block)
* ``forward``        ``parallel/transformer.py:536-577`` (embed, layers, norm, lm_head)
* ``generate_greedy`` ``worker/executor.py:229-347`` with temperature 0
  (prefill with cache, then ``argmax`` of the last position and one-token steps)

Deviations from the reference's composition, all dictated by the workload
being measured (a bf16 embedding and a 4-bit lm_head): the embedding is the
vocab-sharded bf16 gather (``VocabParallelEmbedding``) rather than the
quantized embedding ``ParallelTransformer`` would build, and the lm_head is a
quantized column-parallel linear rather than the dense ``ColumnParallelLinear``
of ``transformer.py:466-475``.

Precision policy (shared with the HIP path): activations are bf16 between ops;
every op computes in fp32 (fp64 accumulation inside quantized matmuls) and
rounds its output once to bf16.  The reference runs the same ops in the
activation dtype under MLX; MLX's per-op rounding is not pinned (parity
unpinned for bit-level agreement; the tests compare within tolerances).

Parity pins: RMSNorm against its closed form on constant rows, RoPE against the
equivalent complex rotation ``(a + ib) * e^{i t theta}`` and its norm
preservation, attention against a per-head scalar loop, GQA against explicit
head sharing, and the incremental KV-cache path against a single full-sequence
forward (both are required by the reference's cache semantics).  The wiring
(``_attn``, ``_mlp``, the block and ``forward``) is pinned by closed forms on
structured weights, each computed in float64 without calling this module:
zero o/down make a block the identity on h; SiLU at known points; gate = 2I,
up = I, down = I give ``silu(2x) * x`` (a swapped gate/up gives
``silu(x) * 2x``); a one-layer model with those weights, o = 0 and an identity
lm_head gives ``norm(h + silu(2 xn) xn)`` with ``xn = norm(h)`` (a post-norm
block, a dropped residual or a missing final norm each miss it by far more
than the tolerance); v = I, o = I give each query head its kv head's input
slice at one token, and q = 0 gives causal running means of v over a prompt.
"""
from dataclasses import dataclass, field

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16, round_bf16
from .gather import vocab_gather_bf16
from .mlx_affine import dequantize_f64


@dataclass
class DecoderShape:
    vocab_size: int
    hidden_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    intermediate_size: int
    head_dim: int = 0
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    bits: int = 4
    group_size: int = 64
    activation: str = "silu"       # ParallelMLP's activation name
    gated: bool = True             # gate/up/down (Llama) or up/down (fc1/fc2)

    def __post_init__(self):
        if not self.head_dim:
            self.head_dim = self.hidden_size // self.num_heads


@dataclass
class QLinear:
    """Quantized linear weights: wq uint32 [N, K*bits/32], s/b uint16 bf16 [N, G]."""
    wq: np.ndarray
    scales: np.ndarray
    biases: np.ndarray
    bias: np.ndarray = None
    _w32: np.ndarray = field(default=None, repr=False)

    def dense_f32(self, group_size, bits):
        if self._w32 is None:
            self._w32 = dequantize_f64(self.wq, self.scales, self.biases, group_size,
                                       bits).astype(np.float32)
        return self._w32


def qlinear(x32, lin: QLinear, shape: DecoderShape):
    """bf16-valued fp32 activations [..., K] -> bf16-valued fp32 [..., N]."""
    w = lin.dense_f32(shape.group_size, shape.bits)
    lead = x32.shape[:-1]
    # fp32 GEMM over fp32-dequantized weights: at decoder scale this differs
    # from the fp64 oracle by ~1e-6 relative, far below the bf16 output step.
    y = round_bf16(x32.reshape(-1, x32.shape[-1]).astype(np.float32) @ w.T)
    if lin.bias is not None:
        y = round_bf16(y + bf16_to_f32(lin.bias))
    return y.reshape(lead + (w.shape[0],))


def rms_norm(x32, w_bf16, eps, bias_bf16=None):
    """``(x / sqrt(mean(x*x) + eps)) * w`` in fp32, rounded once to bf16; with a
    LayerNorm-style bias (``transformer.py:57-59``) the bias is added to that bf16 row
    and the sum rounded again."""
    x = x32.astype(np.float32)
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    y = round_bf16((x / np.sqrt(ms + np.float32(eps))) * bf16_to_f32(w_bf16))
    if bias_bf16 is not None:
        y = round_bf16(y + bf16_to_f32(bias_bf16))
    return y


def rope_cos_sin(positions, head_dim, base):
    """fp32 cos/sin tables [len(positions), head_dim] (both halves repeated)."""
    inv_freq = (np.float32(1.0) /
                (np.float32(base) ** (np.arange(0, head_dim, 2, dtype=np.float32) /
                                      np.float32(head_dim)))).astype(np.float32)
    t = np.asarray(positions, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    cos = np.cos(freqs).astype(np.float32)
    sin = np.sin(freqs).astype(np.float32)
    return np.concatenate([cos, cos], -1), np.concatenate([sin, sin], -1)


def apply_rope(x32, cos, sin):
    """x [B, H, S, D] bf16-valued; rotate-half ``x*cos + [-x2, x1]*sin`` -> bf16."""
    d = x32.shape[-1]
    x1, x2 = x32[..., : d // 2], x32[..., d // 2:]
    rot = np.concatenate([-x2, x1], axis=-1)
    return round_bf16(x32 * cos[None, None] + rot * sin[None, None])


def silu(x32):
    """``x * sigmoid(x)`` (``parallel/mlp.py:161-162``) in fp32, as ``x / (1 + exp(-x))``."""
    x = np.asarray(x32, dtype=np.float32)
    with np.errstate(over="ignore"):
        return x / (np.float32(1) + np.exp(-x, dtype=np.float32))


def activation(x32, name):
    """The MLP activations of ``parallel/mlp.py:159-180`` in fp32 (the op order of
    the formulas there; the GPU kernel follows the same order):

    * ``silu`` / ``swish``: ``x / (1 + exp(-x))`` (= ``x * sigmoid(x)``)
    * ``gelu``:        ``x / (1 + exp(-1.702 x))`` (= ``x * sigmoid(1.702 x)``)
    * ``gelu_new``:    ``0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3)))``
    * ``relu``:        ``max(x, 0)``, NaN kept (``mx.maximum``)
    * ``gelu_exact``:  ``0.5 x (1 + erf(x / sqrt(2)))``
    """
    x = np.asarray(x32, dtype=np.float32)
    f = np.float32
    with np.errstate(over="ignore", invalid="ignore"):
        if name in ("silu", "swish"):
            return silu(x)
        if name == "gelu":
            return x / (f(1) + np.exp(f(-1.702) * x, dtype=np.float32))
        if name == "gelu_new":
            t = np.tanh(f(0.7978845608028654) * (x + f(0.044715) * ((x * x) * x)), dtype=np.float32)
            return (f(0.5) * x) * (f(1) + t)
        if name == "relu":
            return np.where((x > 0) | np.isnan(x), x, f(0))
        if name == "gelu_exact":
            from scipy.special import erf
            e = erf(x * f(0.7071067811865476)).astype(np.float32)
            return (f(0.5) * x) * (f(1) + e)
    raise ValueError(f"Unknown activation: {name}")


def attention_core(q, k, v, scale, causal_offset, mask=None):
    """q [B,H,S,D]; k,v [B,H,T,D] (already GQA-expanded) -> [B,H,S,D] bf16-valued.

    Query row i may attend to key j iff ``j <= i + causal_offset`` (with
    ``causal_offset = T - S`` this is the reference's ``triu(k = T - S + 1)``).
    ``mask``: an additive mask broadcastable to [B,H,S,T], added to the scaled
    scores before the causal mask (``parallel/attention.py:447-458``).
    """
    s = np.einsum("bhsd,bhtd->bhst", q.astype(np.float32), k.astype(np.float32),
                  dtype=np.float32) * np.float32(scale)
    if mask is not None:
        s = s + np.asarray(mask, np.float32)
    S, T = s.shape[-2], s.shape[-1]
    if S > 1:
        i = np.arange(S)[:, None]
        j = np.arange(T)[None, :]
        s = np.where(j <= i + causal_offset, s, np.float32(-np.inf))
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s, dtype=np.float32)
    p = p / p.sum(axis=-1, keepdims=True, dtype=np.float32)
    o = np.einsum("bhst,bhtd->bhsd", p, v.astype(np.float32), dtype=np.float32)
    return round_bf16(o)


class OracleDecoder:
    """numpy restatement of ``ParallelTransformer`` at world_size = 1.

    ``weights`` keys: ``embed`` (uint16 [V, H]), ``norm`` (uint16 [H]),
    ``lm_head`` (QLinear), and ``layers``: list of dicts with ``input_ln``,
    ``post_ln`` (uint16 [H]) and QLinear ``q, k, v, o, gate, up, down``.
    """

    def __init__(self, shape: DecoderShape, weights):
        self.shape = shape
        self.w = weights
        self.reset()

    def reset(self):
        self.cache = [None] * self.shape.num_layers

    def _attn(self, li, x, L, mask=None):
        sh = self.shape
        B, S, _ = x.shape
        D, H, Hk = sh.head_dim, sh.num_heads, sh.num_kv_heads
        q = qlinear(x, L["q"], sh).reshape(B, S, H, D).transpose(0, 2, 1, 3)
        k = qlinear(x, L["k"], sh).reshape(B, S, Hk, D).transpose(0, 2, 1, 3)
        v = qlinear(x, L["v"], sh).reshape(B, S, Hk, D).transpose(0, 2, 1, 3)
        past = self.cache[li]
        off = 0 if past is None else past[0].shape[2]
        cos, sin = rope_cos_sin(np.arange(off, off + S), D, sh.rope_theta)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
        if past is not None:
            k = np.concatenate([past[0], k], axis=2)
            v = np.concatenate([past[1], v], axis=2)
        self.cache[li] = (k, v)
        rep = H // Hk
        kk = np.repeat(k, rep, axis=1)
        vv = np.repeat(v, rep, axis=1)
        o = attention_core(q, kk, vv, 1.0 / np.sqrt(D), k.shape[2] - S, mask=mask)
        o = o.transpose(0, 2, 1, 3).reshape(B, S, H * D)
        return qlinear(o, L["o"], sh)

    def _mlp(self, x, L):
        sh = self.shape
        u = qlinear(x, L["up"], sh)
        if sh.gated:
            g = qlinear(x, L["gate"], sh)
            a = round_bf16(activation(g, sh.activation) * u)
        else:
            a = round_bf16(activation(u, sh.activation))
        return qlinear(a, L["down"], sh)

    def forward(self, ids, last_only=False, mask=None):
        """ids int [B, S] -> logits bf16-valued fp32 [B, S or 1, V]; updates the cache.
        ``mask``: the additive attention mask every layer adds to its scores
        (``transformer.py:548-553``)."""
        sh = self.shape
        ids = np.asarray(ids)
        h = bf16_to_f32(vocab_gather_bf16(ids, self.w["embed"], 0))
        for li, L in enumerate(self.w["layers"]):
            xn = rms_norm(h, L["input_ln"], sh.rms_norm_eps, L.get("input_ln_bias"))
            h = round_bf16(h + self._attn(li, xn, L, mask=mask))
            xn = rms_norm(h, L["post_ln"], sh.rms_norm_eps, L.get("post_ln_bias"))
            h = round_bf16(h + self._mlp(xn, L))
        if last_only:
            h = h[:, -1:]
        hn = rms_norm(h, self.w["norm"], sh.rms_norm_eps, self.w.get("norm_bias"))
        return qlinear(hn, self.w["lm_head"], sh)

    def generate_greedy(self, ids, max_new_tokens, forced=None):
        """Greedy decode (``executor.py:267-325`` at temperature 0).

        Returns (tokens [B, S + n], per-step last-position logits list).  With
        ``forced`` (int [B, n]) the oracle is teacher-forced: it feeds the given
        tokens instead of its own argmax, so its logits can be compared step by
        step with another implementation's run.
        """
        self.reset()
        ids = np.asarray(ids)
        logits = self.forward(ids, last_only=True)
        out = [ids]
        steps = []
        for t in range(max_new_tokens):
            last = logits[:, -1, :]
            steps.append(last)
            nxt = np.argmax(last, axis=-1) if forced is None else np.asarray(forced)[:, t]
            out.append(nxt[:, None])
            if t == max_new_tokens - 1:
                break
            logits = self.forward(nxt[:, None], last_only=True)
        return np.concatenate(out, axis=1), steps


def random_decoder_weights(shape: DecoderShape, seed=0, std=0.02):
    """Random-init weights: N(0, std) fp32, quantized (MLX affine) to bits/g.

    Norm weights are 1 + N(0, 0.1) so the norms are not the identity; the
    embedding is N(0, std) rounded to bf16.
    """
    from .mlx_affine import quantize_bf16
    rng = np.random.default_rng(seed)
    H, I = shape.hidden_size, shape.intermediate_size
    D = shape.head_dim

    def ql(n, k):
        w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)
        wq, s, b = quantize_bf16(w, shape.group_size, shape.bits)
        return QLinear(wq, s, b)

    def norm_w():
        return f32_to_bf16(1.0 + 0.1 * rng.standard_normal(H, dtype=np.float32))

    layers = []
    for _ in range(shape.num_layers):
        layers.append(dict(
            input_ln=norm_w(), post_ln=norm_w(),
            q=ql(shape.num_heads * D, H), k=ql(shape.num_kv_heads * D, H),
            v=ql(shape.num_kv_heads * D, H), o=ql(H, shape.num_heads * D),
            gate=ql(I, H), up=ql(I, H), down=ql(H, I)))
    embed = f32_to_bf16(rng.standard_normal((shape.vocab_size, H), dtype=np.float32)
                        * np.float32(std))
    return dict(embed=embed, norm=norm_w(), lm_head=ql(shape.vocab_size, H), layers=layers)
