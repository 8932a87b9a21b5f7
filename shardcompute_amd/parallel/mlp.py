"""Tensor-parallel MLP over the HIP kernels.

Drop-in for ``ParallelMLP`` of ``src/shardcompute/parallel/mlp.py:18-279``:
gated, ``down(f(gate(x)) * up(x))``; ungated, ``down(f(up(x)))`` (``:228-254``),
with f any activation the reference accepts (``silu``/``swish``, ``gelu``,
``gelu_new``, ``relu``, ``gelu_exact``, ``:159-180``).  gate and up run as one
fused quantized product (bit-identical per column); the gated SiLU, the Llama
family's MLP, applies silu(gate) * up inside that product's kernel; every other
form runs the product, ``sc_act_bf16`` and the row-parallel down projection
(all-reduce = identity at world_size 1).
"""
import logging
from typing import Optional

import torch

from .. import _lib
from ._fused import FusedColumns
from .column_linear import ColumnParallelLinear
from .quantized_linear import QuantizedColumnParallelLinear, QuantizedRowParallelLinear
from .row_linear import RowParallelLinear

logger = logging.getLogger(__name__)

_SUPPORTED = ("silu", "swish")


class ParallelMLP:
    def __init__(self, hidden_size: int, intermediate_size: int, world_size: int, rank: int, communicator=None,
                 activation: str = "silu", bias: bool = False, use_gated: bool = True, use_quantized: bool = False,
                 quantization_bits: int = 4, quantization_group_size: int = 64, device=None):
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.world_size = world_size
        self.rank = rank
        self.communicator = communicator
        self.use_gated = use_gated
        self.use_quantized = use_quantized
        if intermediate_size % world_size != 0:
            raise ValueError(f"intermediate_size ({intermediate_size}) must be divisible by "
                             f"world_size ({world_size})")
        self.local_intermediate = intermediate_size // world_size
        self.activation_name = activation
        if activation not in _SUPPORTED and activation not in ("gelu", "gelu_new", "relu", "gelu_exact"):
            raise ValueError(f"Unknown activation: {activation}")
        if use_quantized:
            def col():
                return QuantizedColumnParallelLinear(hidden_size, intermediate_size, world_size, rank, bias=bias,
                                                     gather_output=False, bits=quantization_bits,
                                                     group_size=quantization_group_size, device=device)
            self.gate_proj = col() if use_gated else None
            self.up_proj = col()
            self.down_proj = QuantizedRowParallelLinear(intermediate_size, hidden_size, world_size, rank, bias=bias,
                                                        input_is_partitioned=True, communicator=communicator,
                                                        bits=quantization_bits, group_size=quantization_group_size,
                                                        device=device)
        else:
            def col():
                return ColumnParallelLinear(hidden_size, intermediate_size, world_size, rank, bias=bias,
                                            gather_output=False, device=device)
            self.gate_proj = col() if use_gated else None
            self.up_proj = col()
            self.down_proj = RowParallelLinear(intermediate_size, hidden_size, world_size, rank, bias=bias,
                                               input_is_partitioned=True, communicator=communicator, device=device)
        self.gate_up = FusedColumns([self.gate_proj, self.up_proj]) if use_gated else None

    def load_shards(self, up_weight, up_bias, down_weight, down_bias, gate_weight=None, gate_bias=None):
        self.up_proj.load_shard_direct(up_weight, up_bias)
        self.down_proj.load_shard_direct(down_weight, down_bias)
        if self.use_gated and gate_weight is not None:
            self.gate_proj.load_shard_direct(gate_weight, gate_bias)

    def load_quantized_shards(self, up_weight, up_scales, up_biases, up_linear_bias, down_weight, down_scales,
                              down_biases, down_linear_bias, gate_weight=None, gate_scales=None, gate_biases=None,
                              gate_linear_bias=None):
        if not self.use_quantized:
            raise RuntimeError("Cannot load quantized shards into non-quantized MLP")
        self.up_proj.load_quantized_shard(up_weight, up_scales, up_biases, up_linear_bias)
        self.down_proj.load_quantized_shard(down_weight, down_scales, down_biases, down_linear_bias)
        if self.use_gated and gate_weight is not None:
            self.gate_proj.load_quantized_shard(gate_weight, gate_scales, gate_biases, gate_linear_bias)

    @property
    def fused_swiglu(self) -> bool:
        """The gated SiLU MLP: its gate|up product applies the activation itself."""
        return self.use_gated and self.activation_name in _SUPPORTED

    def intermediate(self, x2, gu_out=None, out=None):
        """f(gate(x)) * up(x) (gated) or f(up(x)) for x2 ``[rows, hidden]`` ->
        ``[rows, local_intermediate]``."""
        if self.use_gated:
            gu = self.gate_up(x2, out=gu_out)
            return _lib.act(gu, self.activation_name, gated=True, out=out)
        return _lib.act(self.up_proj.forward_sync(x2), self.activation_name, gated=False, out=out)

    def act_call(self, h, norm, residual=None, h_out=None, xn_out=None, act_out=None, gu_out=None):
        """The activation of the MLP's input projections applied to norm(h + residual)
        (``transformer.py:249-253``); the residual sum goes to ``h_out``.  The gated SiLU
        with a bias-free norm runs as one kernel (norm, gate|up, SiLU gate)."""
        if self.fused_swiglu:
            return self.gate_up.swiglu_call(h, norm, residual=residual, h_out=h_out, xn_out=xn_out,
                                            act_out=act_out, gu_out=gu_out)
        xn = norm(h, residual=residual, h_out=h_out, out=xn_out)
        return self.intermediate(xn, gu_out=gu_out, out=act_out)

    def act_from_xn(self, xn, act_out=None, gu_out=None):
        """The activation of the input projections of an already normalised input
        (the gated SiLU applied inside the gate|up product)."""
        if self.fused_swiglu:
            return self.gate_up.swiglu_call(xn, None, act_out=act_out, gu_out=gu_out)
        return self.intermediate(xn, gu_out=gu_out, out=act_out)

    async def down_from_gate_up(self, gate_up, act_out=None):
        """down(f(gate) * up) from the fused gate|up product (gated MLPs)."""
        if not self.use_gated:
            raise ValueError("down_from_gate_up needs a gated MLP")
        return await self.down_proj.forward(_lib.act(gate_up, self.activation_name, gated=True, out=act_out))

    async def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        lead = hidden_states.shape[:-1]
        a = self.intermediate(hidden_states.reshape(-1, self.hidden_size))
        out = await self.down_proj.forward(a)
        return out.reshape(*lead, self.hidden_size)

    def forward_sync_partial(self, hidden_states: torch.Tensor) -> torch.Tensor:
        lead = hidden_states.shape[:-1]
        a = self.intermediate(hidden_states.reshape(-1, self.hidden_size))
        return self.down_proj.forward_partial(a).reshape(*lead, self.hidden_size)

    @property
    def num_parameters(self) -> int:
        params = self.up_proj.num_parameters + self.down_proj.num_parameters
        if self.gate_proj is not None:
            params += self.gate_proj.num_parameters
        return params
