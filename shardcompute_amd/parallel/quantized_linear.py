"""Quantized tensor-parallel linears over the HIP fused dequant kernels.

Drop-in for ``src/shardcompute/parallel/quantized_linear.py``: same constructor
arguments, attributes, load methods, ``async forward`` / ``forward_sync`` /
``forward_partial`` / ``add_bias`` and errors.  Weights are torch-ROCm device
tensors: ``quantized_weight`` uint32 ``[local_out, in * bits / 32]`` (column) or
``[out, local_in * bits / 32]`` (row), ``scales`` / ``biases_quant`` bf16
``[rows, cols / group_size]``.  Every matmul is one ``sc_qmm_bf16`` call (the
reference's ``mx.quantized_matmul(..., transpose=True)`` plus the bias add).
"""
import logging
from typing import Optional

import torch

from .. import _lib
from ..communicator import IdentityCommunicator
from ._tensors import default_device, nbytes, packed, to_device

logger = logging.getLogger(__name__)


def _quantize_shard(weight_shard, bits, group_size, device):
    """``mx.quantize(weight.astype(float32), group_size, bits)`` on the GPU."""
    w = to_device(weight_shard, device, torch.float32)
    return _lib.quantize(w, bits=bits, group_size=group_size)


class QuantizedColumnParallelLinear:
    """Column-parallel linear with MLX-affine quantized weights.

    Reference: ``parallel/quantized_linear.py:17-251``.  Holds output columns
    ``[col_start, col_end)``; ``forward`` optionally all-gathers the output.
    """

    def __init__(self, in_features: int, out_features: int, world_size: int, rank: int, bias: bool = True,
                 gather_output: bool = False, communicator=None, group_size: int = 64, bits: int = 4,
                 device: Optional[torch.device] = None):
        self.in_features = in_features
        self.out_features = out_features
        self.world_size = world_size
        self.rank = rank
        self.gather_output = gather_output
        self.communicator = communicator
        self.group_size = group_size
        self.bits = bits
        if out_features % world_size != 0:
            raise ValueError(f"out_features ({out_features}) must be divisible by world_size ({world_size})")
        self.local_out_features = out_features // world_size
        self.col_start = rank * self.local_out_features
        self.col_end = self.col_start + self.local_out_features
        self.quantized_weight: Optional[torch.Tensor] = None
        self.scales: Optional[torch.Tensor] = None
        self.biases_quant: Optional[torch.Tensor] = None
        self.bias: Optional[torch.Tensor] = None
        self.has_bias = bias
        self._device = device

    @property
    def device(self):
        if self._device is None:
            self._device = default_device()
        return self._device

    def load_shard_and_quantize(self, weight_shard, bias_shard=None):
        """Quantize a pre-sharded full-precision weight ``[in_features, local_out_features]``.

        Mirrors ``quantized_linear.py:96-125``: the shard is quantized as given
        (groups along its last dimension) and later used with ``transpose=True``,
        exactly as the reference does.
        """
        expected = (self.in_features, self.local_out_features)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}")
        self.quantized_weight, self.scales, self.biases_quant = _quantize_shard(
            weight_shard, self.bits, self.group_size, self.device)
        if self.has_bias and bias_shard is not None:
            self.bias = to_device(bias_shard, self.device, torch.bfloat16)

    def load_quantized_shard(self, quantized_weight, scales, biases, linear_bias=None):
        """Load pre-quantized weights (``quantized_linear.py:127-150``)."""
        self.quantized_weight = packed(quantized_weight, self.device)
        self.scales = to_device(scales, self.device, torch.bfloat16)
        self.biases_quant = to_device(biases, self.device, torch.bfloat16)
        if self.has_bias and linear_bias is not None:
            self.bias = to_device(linear_bias, self.device, torch.bfloat16)

    def _qmm(self, x, bias):
        return _lib.qmm(x, self.quantized_weight, self.scales, self.biases_quant, bias=bias, bits=self.bits,
                        group_size=self.group_size)

    async def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.quantized_weight is None:
            raise RuntimeError("Weight not loaded. Call load_shard_and_quantize() first.")
        output = self._qmm(x, self.bias if self.has_bias else None)
        if self.gather_output:
            if self.communicator is None:
                raise RuntimeError("Communicator required for gather_output=True")
            output = await self.communicator.all_gather(output, dim=-1)
        return output

    def forward_sync(self, x: torch.Tensor) -> torch.Tensor:
        if self.quantized_weight is None:
            raise RuntimeError("Weight not loaded")
        return self._qmm(x, self.bias if self.has_bias else None)

    @property
    def num_parameters(self) -> int:
        params = self.in_features * self.local_out_features
        if self.has_bias:
            params += self.local_out_features
        return params

    @property
    def memory_bytes(self) -> int:
        if self.quantized_weight is None:
            return 0
        return (nbytes(self.quantized_weight) + nbytes(self.scales) + nbytes(self.biases_quant)
                + nbytes(self.bias))

    def __repr__(self) -> str:
        return (f"QuantizedColumnParallelLinear(in_features={self.in_features}, out_features={self.out_features}, "
                f"local_out_features={self.local_out_features}, rank={self.rank}/{self.world_size}, "
                f"bits={self.bits})")


class QuantizedRowParallelLinear:
    """Row-parallel linear with MLX-affine quantized weights.

    Reference: ``parallel/quantized_linear.py:254-518``.  Holds input rows
    ``[row_start, row_end)``; ``forward`` = partial qmm -> all-reduce(sum) ->
    bias (rank 0 only).  With no communicator (world_size 1, or one rank's
    shard measured on its own) the all-reduce is the identity.
    """

    def __init__(self, in_features: int, out_features: int, world_size: int, rank: int, bias: bool = True,
                 input_is_partitioned: bool = True, communicator=None, group_size: int = 64, bits: int = 4,
                 device: Optional[torch.device] = None):
        self.in_features = in_features
        self.out_features = out_features
        self.world_size = world_size
        self.rank = rank
        self.input_is_partitioned = input_is_partitioned
        self.communicator = communicator
        self.group_size = group_size
        self.bits = bits
        if in_features % world_size != 0:
            raise ValueError(f"in_features ({in_features}) must be divisible by world_size ({world_size})")
        self.local_in_features = in_features // world_size
        self.row_start = rank * self.local_in_features
        self.row_end = self.row_start + self.local_in_features
        self.quantized_weight: Optional[torch.Tensor] = None
        self.scales: Optional[torch.Tensor] = None
        self.biases_quant: Optional[torch.Tensor] = None
        self.bias: Optional[torch.Tensor] = None
        self.has_bias = bias
        self._device = device

    @property
    def device(self):
        if self._device is None:
            self._device = default_device()
        return self._device

    def load_shard_and_quantize(self, weight_shard, bias_shard=None):
        """Quantize ``[local_in_features, out_features]`` (``quantized_linear.py:333-363``)."""
        expected = (self.local_in_features, self.out_features)
        if tuple(weight_shard.shape) != expected:
            raise ValueError(f"Weight shard shape {tuple(weight_shard.shape)} doesn't match expected {expected}")
        self.quantized_weight, self.scales, self.biases_quant = _quantize_shard(
            weight_shard, self.bits, self.group_size, self.device)
        if self.has_bias and bias_shard is not None and self.rank == 0:
            self.bias = to_device(bias_shard, self.device, torch.bfloat16)

    def load_quantized_shard(self, quantized_weight, scales, biases, linear_bias=None):
        """Load pre-quantized weights; slice full-width scales/biases to this shard.

        Mirrors ``quantized_linear.py:365-417``: when the weight is
        ``[out_features, local_in * bits / 32]`` but scales/biases carry the
        groups of every rank (``world_size`` times the local count), keep this
        rank's column range of them; otherwise leave them unchanged (with the
        reference's warnings).
        """
        self.quantized_weight = packed(quantized_weight, self.device)
        self.scales = to_device(scales, self.device, torch.bfloat16)
        self.biases_quant = to_device(biases, self.device, torch.bfloat16)
        if (self.quantized_weight is not None and self.scales is not None and self.scales.dim() == 2
                and self.quantized_weight.shape[0] == self.out_features):
            pack_factor = 32 // self.bits
            input_shard = self.quantized_weight.shape[1] * pack_factor
            if input_shard % self.group_size == 0:
                expected_groups = input_shard // self.group_size
                full_groups = self.scales.shape[1]
                if full_groups == expected_groups * self.world_size:
                    start = self.rank * expected_groups
                    end = start + expected_groups
                    self.scales = self.scales[:, start:end].contiguous()
                    if self.biases_quant is not None and self.biases_quant.dim() == 2:
                        self.biases_quant = self.biases_quant[:, start:end].contiguous()
                elif full_groups != expected_groups:
                    logger.warning(f"QuantizedRowParallelLinear scales shape {tuple(self.scales.shape)} does not "
                                   f"match expected groups {expected_groups}; leaving scales/biases unchanged")
            else:
                logger.warning(f"QuantizedRowParallelLinear input shard {input_shard} not divisible by "
                               f"group_size {self.group_size}; leaving scales/biases unchanged")
        if self.has_bias and linear_bias is not None and self.rank == 0:
            self.bias = to_device(linear_bias, self.device, torch.bfloat16)

    def _qmm(self, x, bias=None):
        return _lib.qmm(x, self.quantized_weight, self.scales, self.biases_quant, bias=bias, bits=self.bits,
                        group_size=self.group_size)

    async def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.quantized_weight is None:
            raise RuntimeError("Weight not loaded")
        if self.communicator is None or isinstance(self.communicator, IdentityCommunicator):
            # identity all-reduce: bf16(partial) + bias is what the kernel epilogue computes
            return self._qmm(x, self.bias if self.has_bias else None)
        output = await self.communicator.all_reduce(self._qmm(x), op="sum")
        return self.add_bias(output)

    def forward_partial(self, x: torch.Tensor) -> torch.Tensor:
        if self.quantized_weight is None:
            raise RuntimeError("Weight not loaded")
        return self._qmm(x)

    @property
    def folds_norm(self) -> bool:
        """Whether forward_add_norm runs as one fused call: the all-reduce between the
        product and the residual add is the identity."""
        return self.communicator is None or isinstance(self.communicator, IdentityCommunicator)

    def forward_add_norm(self, x, residual, norm, h_out=None, xn_out=None):
        """(h, xn) = (forward(x) + residual, norm(h)) for a bias-free RMSNorm, the
        product's split-K pass folded into the norm's (one launch fewer; the same
        bits as forward followed by the norm).  Only with an identity all-reduce."""
        if self.quantized_weight is None:
            raise RuntimeError("Weight not loaded")
        if not self.folds_norm or not norm.fusable:
            raise ValueError("forward_add_norm needs an identity all-reduce and a bias-free norm")
        norm._check()
        return _lib.qmm_add_rmsnorm(x, self.quantized_weight, self.scales, self.biases_quant, residual, norm.weight,
                                    norm.eps, bias=self.bias if self.has_bias else None, bits=self.bits,
                                    group_size=self.group_size, h_out=h_out, xn_out=xn_out)

    def add_bias(self, x: torch.Tensor) -> torch.Tensor:
        if self.has_bias and self.bias is not None:
            return (x.float() + self.bias.float()).to(x.dtype)
        return x

    @property
    def num_parameters(self) -> int:
        params = self.local_in_features * self.out_features
        if self.has_bias and self.rank == 0:
            params += self.out_features
        return params

    @property
    def memory_bytes(self) -> int:
        if self.quantized_weight is None:
            return 0
        return (nbytes(self.quantized_weight) + nbytes(self.scales) + nbytes(self.biases_quant)
                + nbytes(self.bias))

    def __repr__(self) -> str:
        return (f"QuantizedRowParallelLinear(in_features={self.in_features}, out_features={self.out_features}, "
                f"local_in_features={self.local_in_features}, rank={self.rank}/{self.world_size}, "
                f"bits={self.bits})")
