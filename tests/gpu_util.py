"""Helpers shared by the GPU tests: numpy <-> torch-ROCm conversions and metrics."""
import numpy as np
import torch

from oracle.bf16 import bf16_to_f32

# Linear outputs (bf16 out, fp32 accumulate) must be within this max-abs-rel
# error of the oracle:  max|y - ref| / max|ref|.
LINEAR_TOL = 1e-2


def dev_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).cuda()


def dev_u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32).cuda()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host_u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def host_u32(t):
    return t.detach().cpu().contiguous().view(torch.int32).numpy().view(np.uint32)


def max_abs_rel(y_u16, ref_u16):
    y = bf16_to_f32(y_u16).astype(np.float64)
    r = bf16_to_f32(ref_u16).astype(np.float64) if ref_u16.dtype == np.uint16 else ref_u16.astype(np.float64)
    denom = np.max(np.abs(r))
    return float(np.max(np.abs(y - r)) / (denom if denom > 0 else 1.0))


def bf16_ulp_diff(a_u16, b_u16):
    """Distance in bf16 steps between two arrays of finite bf16 patterns."""
    def ordered(u):
        u = u.astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), 0x8000 + u)
    return np.abs(ordered(a_u16) - ordered(b_u16))
