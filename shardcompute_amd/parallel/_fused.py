"""Column concatenation of projections that read the same input.

q/k/v (``parallel/attention.py:406-408``) and gate/up (``parallel/mlp.py:241-242``)
are separate column-parallel linears in the reference.  Each output column of a
linear depends only on its own weight row, so stacking the rows of several
linears into one matrix gives bit-identical outputs in a single launch: one
weight stream instead of three (or two), which is what a bandwidth-bound decode
GEMV wants.  After fusing, the parts' tensors become row views of the fused
buffers, so no weight is stored twice; reloading a part is noticed (its tensor
no longer points where it did) and the fused matrix is rebuilt on the next call.
"""
import torch

from .. import _lib


class FusedColumns:
    def __init__(self, parts):
        self.parts = list(parts)
        self.quantized = None
        self._wq = self._s = self._b = self._w = self._bias = None
        self._rows = []

    @property
    def widths(self):
        return [p.local_out_features for p in self.parts]

    @property
    def out_features(self):
        return sum(self.widths)

    def _part_ptrs(self):
        if self.quantized:
            return tuple((p.quantized_weight.data_ptr(), p.scales.data_ptr(), p.biases_quant.data_ptr(),
                          None if p.bias is None else p.bias.data_ptr()) for p in self.parts)
        return tuple((p.weight.data_ptr(), None if p.bias is None else p.bias.data_ptr()) for p in self.parts)

    def _current(self):
        if self.quantized is None:
            return False
        try:
            return self._part_ptrs() == self._src
        except AttributeError:   # a part lost its weights
            return False

    def build(self):
        ps = self.parts
        quantized = hasattr(ps[0], "quantized_weight")
        if quantized:
            if any(p.quantized_weight is None for p in ps):
                raise RuntimeError("Weight not loaded")
            bits = {p.bits for p in ps}
            gs = {p.group_size for p in ps}
            if len(bits) != 1 or len(gs) != 1:
                raise ValueError("fused projections must share bits and group size")
            self.bits, self.group_size = bits.pop(), gs.pop()
            self._wq = torch.cat([p.quantized_weight for p in ps], 0).contiguous()
            self._s = torch.cat([p.scales for p in ps], 0).contiguous()
            self._b = torch.cat([p.biases_quant for p in ps], 0).contiguous()
            r0 = 0
            for p, n in zip(ps, self.widths):
                p.quantized_weight = self._wq[r0:r0 + n]
                p.scales = self._s[r0:r0 + n]
                p.biases_quant = self._b[r0:r0 + n]
                r0 += n
        else:
            if any(p.weight is None for p in ps):
                raise RuntimeError("Weight not loaded")
            # dense weights keep the reference's [in, out] layout; the fused matrix is
            # column-stacked and the parts are not re-pointed (column slices of it
            # would not be contiguous)
            self._w = torch.cat([p.weight for p in ps], 1).contiguous()
        biases = [p.bias if (p.has_bias and p.bias is not None) else None for p in ps]
        if any(b is not None for b in biases):
            dev = (self._wq if quantized else self._w).device
            self._bias = torch.cat([b if b is not None else torch.zeros(n, dtype=torch.bfloat16, device=dev)
                                    for b, n in zip(biases, self.widths)]).contiguous()
        else:
            self._bias = None
        self.quantized = quantized
        self._src = self._part_ptrs()

    def __call__(self, x, out=None):
        if not self._current():
            self.build()
        if self.quantized:
            return _lib.qmm(x, self._wq, self._s, self._b, bias=self._bias, bits=self.bits,
                            group_size=self.group_size, out=out)
        y = x @ self._w
        if self._bias is not None:
            y = y + self._bias
        if out is not None:
            out.copy_(y.reshape(out.shape))
            return out
        return y

    def norm_call(self, h, norm, residual=None, h_out=None, xn_out=None, out=None):
        """The stacked product of ``norm(h + residual)``: the RMSNorm (and residual
        add, written to ``h_out``) runs inside the quantized kernel.  Returns (y, xn)."""
        if not self._current():
            self.build()
        norm._check()
        if self.quantized and norm.fusable:
            return _lib.qmm_rmsnorm(h, norm.weight, norm.eps, self._wq, self._s, self._b, residual=residual,
                                    h_out=h_out, xn_out=xn_out, bias=self._bias, bits=self.bits,
                                    group_size=self.group_size, out=out)
        xn = norm(h, residual=residual, h_out=h_out, out=xn_out)
        return self(xn, out=out), xn

    def swiglu_call(self, h, norm=None, residual=None, h_out=None, xn_out=None, act_out=None, gu_out=None):
        """silu(gate) * up for a gate|up stack, of ``norm(h + residual)`` when a norm is
        given: the quantized kernel pairs each gate column with its up column and
        writes the gated activation directly.  Returns act."""
        if not self._current():
            self.build()
        if len(self.parts) != 2 or self.widths[0] != self.widths[1]:
            raise ValueError("swiglu needs a gate|up pair of equal widths")
        if norm is not None:
            norm._check()
        if self.quantized and (norm is None or norm.fusable):
            act, _ = _lib.qmm_swiglu(h, self._wq, self._s, self._b, norm_weight=norm.weight if norm else None,
                                     eps=norm.eps if norm else 1e-5, residual=residual, h_out=h_out,
                                     xn_out=xn_out, bias=self._bias, bits=self.bits, group_size=self.group_size,
                                     act_out=act_out, gate_up_scratch=gu_out)
            return act
        xn = norm(h, residual=residual, h_out=h_out, out=xn_out) if norm else h
        return _lib.silu_mul(self(xn, out=gu_out), out=act_out)

    def split(self, y):
        return torch.split(y, self.widths, dim=-1)
