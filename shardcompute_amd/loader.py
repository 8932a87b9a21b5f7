"""Per-rank safetensors checkpoints into the parallel layers.

Drop-in for ``detect_parallelism_mode`` and ``ModelLoader`` of
``src/shardcompute/model/loader.py:17-413`` (tensor-parallel mode).  The on-disk
format is the reference's, written by its sharder (``model/sharder.py:57-180``):

* ``<shard_dir>/rank_<r>/model.safetensors`` per rank, ``<shard_dir>/config.json``
  optionally naming the parallelism mode;
* Hugging Face key names (``model.layers.<i>.self_attn.q_proj.weight`` ...), with
  Phi-2 variants (``self_attn.dense``, ``mlp.fc1`` / ``mlp.fc2``,
  ``model.final_layernorm``) and optional linear / layernorm ``.bias`` keys;
* dense 2-D linears already transposed to ``[in, out]`` and split (column-parallel
  along out, row-parallel along in); quantized linears as MLX affine triples
  ``.weight`` (uint32 ``[out, in * bits / 32]``), ``.scales`` and ``.biases``
  (``[out, in / group]``, fp32 or bf16), split along the same dims, row-parallel
  scales possibly left full width (the layer slices them, ``quantized_linear.py:385-414``).

Tensors are read with safetensors' torch backend straight onto the model's device
(no host-side copy of the whole checkpoint).  A checkpoint that stores bf16 values
as 16-bit unsigned integers (bit patterns) is accepted too.
"""
import json
import logging
from pathlib import Path
from typing import Dict, Optional

import torch
from safetensors import safe_open

logger = logging.getLogger(__name__)


def detect_parallelism_mode(shard_dir: Path) -> str:
    """``"tensor"`` or ``"pipeline"`` from ``config.json``'s ``parallel.mode``
    (``loader.py:17-33``); ``"tensor"`` when the file or field is absent."""
    config_path = Path(shard_dir) / "config.json"
    if config_path.exists():
        with open(config_path) as f:
            data = json.load(f)
        return data.get("parallel", {}).get("mode", "tensor")
    return "tensor"


def _as_model_tensor(t: torch.Tensor) -> torch.Tensor:
    """16-bit unsigned tensors are bf16 bit patterns; everything else as stored."""
    if t.dtype == torch.uint16:
        return t.view(torch.bfloat16)
    return t


class ModelLoader:
    """Loads one rank's shard file into a ``ParallelTransformer``."""

    # Hugging Face name -> layer attribute (``loader.py:43-64``; documentation of
    # the mapping the methods below apply, kept for callers that read it)
    WEIGHT_MAP = {
        "model.embed_tokens.weight": "embed_tokens",
        "lm_head.weight": "lm_head",
        "model.norm.weight": "norm",
        "model.layers.{layer}.input_layernorm.weight": "layers.{layer}.input_layernorm",
        "model.layers.{layer}.post_attention_layernorm.weight": "layers.{layer}.post_attention_layernorm",
        "model.layers.{layer}.self_attn.q_proj.weight": "layers.{layer}.attention.q_proj",
        "model.layers.{layer}.self_attn.k_proj.weight": "layers.{layer}.attention.k_proj",
        "model.layers.{layer}.self_attn.v_proj.weight": "layers.{layer}.attention.v_proj",
        "model.layers.{layer}.self_attn.o_proj.weight": "layers.{layer}.attention.o_proj",
        "model.layers.{layer}.mlp.gate_proj.weight": "layers.{layer}.mlp.gate_proj",
        "model.layers.{layer}.mlp.up_proj.weight": "layers.{layer}.mlp.up_proj",
        "model.layers.{layer}.mlp.down_proj.weight": "layers.{layer}.mlp.down_proj",
    }

    def __init__(self, rank: int, world_size: int, quantized: bool = False):
        self.rank = rank
        self.world_size = world_size
        self.quantized = quantized

    @staticmethod
    def detect_quantization(shard_dir: Path, rank: int = 0) -> bool:
        """True when the rank's file holds both ``.scales`` and ``.biases`` keys
        (``loader.py:80-104``)."""
        model_file = Path(shard_dir) / f"rank_{rank}" / "model.safetensors"
        if not model_file.exists():
            return False
        with safe_open(str(model_file), framework="pt") as f:
            keys = list(f.keys())
        return any(".scales" in k for k in keys) and any(".biases" in k for k in keys)

    async def load_shards(self, model, shard_dir: Path):
        """Load ``rank_<rank>/model.safetensors`` into ``model`` (``loader.py:106-131``)."""
        rank_dir = Path(shard_dir) / f"rank_{self.rank}"
        if not rank_dir.exists():
            raise FileNotFoundError(f"Shard directory not found: {rank_dir}")
        weights = self._load_safetensors(rank_dir / "model.safetensors", getattr(model, "device", None))
        self._load_embedding(model, weights)
        self._load_layers(model, weights)
        self._load_norm(model, weights)
        self._load_lm_head(model, weights)
        logger.info(f"Rank {self.rank} loaded model weights from {shard_dir}")

    def _load_safetensors(self, path: Path, device=None) -> Dict[str, torch.Tensor]:
        """Every tensor of the file, read onto ``device`` (host memory when None)."""
        weights = {}
        dev = "cpu" if device is None else str(device)
        with safe_open(str(path), framework="pt", device=dev) as f:
            for key in f.keys():
                weights[key] = _as_model_tensor(f.get_tensor(key))
        return weights

    # ---------------------------------------------------------------- pieces

    def _load_embedding(self, model, weights):
        """``loader.py:142-170``: first of the usual names; quantized when this
        loader is and the file has the scales and biases."""
        for key in ("model.embed_tokens.weight", "embed_tokens.weight", "wte.weight"):
            if key in weights:
                base = key.rsplit(".weight", 1)[0]
                scales, biases = weights.get(f"{base}.scales"), weights.get(f"{base}.biases")
                if self.quantized and scales is not None and biases is not None:
                    model.load_quantized_embedding_weights(weights[key], scales, biases)
                else:
                    model.embed_tokens.load_shard_direct(weights[key])
                return

    def _load_norm(self, model, weights):
        """``loader.py:172-195``: Llama ``norm``, Phi ``final_layernorm``, GPT ``ln_f``."""
        for key in ("model.norm.weight", "model.final_layernorm.weight", "norm.weight", "ln_f.weight"):
            if key in weights:
                model.norm.load_weights(weights[key], weights.get(key.replace(".weight", ".bias")))
                return

    def _load_lm_head(self, model, weights):
        """``loader.py:197-212``; a quantized lm_head (``.scales``/``.biases`` in the
        file and a quantized head in the model) loads as a quantized shard."""
        lm = getattr(model, "lm_head", None)
        if lm is None or "lm_head.weight" not in weights:
            return
        weight, bias = weights["lm_head.weight"], weights.get("lm_head.bias")
        scales, biases = weights.get("lm_head.scales"), weights.get("lm_head.biases")
        if scales is not None and biases is not None and hasattr(lm, "load_quantized_shard"):
            lm.load_quantized_shard(weight, scales, biases, bias)
        else:
            lm.load_shard_direct(weight, bias)

    def _load_layers(self, model, weights):
        for layer_idx, layer in enumerate(model.layers):
            self._load_single_layer(layer_idx, layer, weights)

    def _load_single_layer(self, layer_idx: int, layer, weights):
        """One decoder layer (``loader.py:224-413``)."""
        prefix = f"model.layers.{layer_idx}"
        ln_key, ln_bias = f"{prefix}.input_layernorm.weight", f"{prefix}.input_layernorm.bias"
        post_key, post_bias = f"{prefix}.post_attention_layernorm.weight", f"{prefix}.post_attention_layernorm.bias"
        if ln_key in weights:
            layer.input_layernorm.load_weights(weights[ln_key], weights.get(ln_bias))
        if post_key in weights:
            layer.post_attention_layernorm.load_weights(weights[post_key], weights.get(post_bias))
        elif ln_key in weights:
            # parallel attention + MLP (Phi-2): both read the input layernorm
            layer.post_attention_layernorm.load_weights(weights[ln_key], weights.get(ln_bias))

        self._load_attention(prefix, layer, weights)
        self._load_mlp(prefix, layer, weights)

    def _load_attention(self, prefix: str, layer, weights):
        att = f"{prefix}.self_attn"
        o_name = "o_proj" if f"{att}.o_proj.weight" in weights else "dense"
        names = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "o": o_name}
        present = {p: f"{att}.{n}.weight" in weights for p, n in names.items()}
        if not any(present.values()):
            return

        def part(p, suffix):
            return weights.get(f"{att}.{names[p]}.{suffix}")

        if self.quantized and f"{att}.q_proj.scales" in weights:
            kwargs = {}
            for p in ("q", "k", "v", "o"):
                kwargs[f"{p}_weight"] = part(p, "weight")
                kwargs[f"{p}_scales"] = part(p, "scales")
                kwargs[f"{p}_biases"] = part(p, "biases")
                kwargs[f"{p}_linear_bias"] = part(p, "bias")
            layer.attention.load_quantized_shards(**kwargs)
        else:
            layer.attention.load_shards(**{f"{p}_{s}": part(p, "weight" if s == "weight" else "bias")
                                           for p in ("q", "k", "v", "o") for s in ("weight", "bias")})

    def _load_mlp(self, prefix: str, layer, weights):
        mlp = f"{prefix}.mlp"
        if f"{mlp}.gate_proj.weight" in weights:
            names = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}
        elif f"{mlp}.fc1.weight" in weights:
            names = {"gate": None, "up": "fc1", "down": "fc2"}     # Phi-2: ungated
        else:
            return

        def part(p, suffix) -> Optional[torch.Tensor]:
            return None if names[p] is None else weights.get(f"{mlp}.{names[p]}.{suffix}")

        quantized_file = any(f"{mlp}.{n}.scales" in weights for n in ("up_proj", "gate_proj", "fc1"))
        if self.quantized and quantized_file:
            layer.mlp.load_quantized_shards(
                up_weight=part("up", "weight"), up_scales=part("up", "scales"), up_biases=part("up", "biases"),
                up_linear_bias=part("up", "bias"),
                down_weight=part("down", "weight"), down_scales=part("down", "scales"),
                down_biases=part("down", "biases"), down_linear_bias=part("down", "bias"),
                gate_weight=part("gate", "weight"), gate_scales=part("gate", "scales"),
                gate_biases=part("gate", "biases"), gate_linear_bias=part("gate", "bias"))
        else:
            layer.mlp.load_shards(up_weight=part("up", "weight"), up_bias=part("up", "bias"),
                                  down_weight=part("down", "weight"), down_bias=part("down", "bias"),
                                  gate_weight=part("gate", "weight"), gate_bias=part("gate", "bias"))
