"""Conversions of caller-supplied weights into device tensors of the layout the
HIP library expects (bf16 activations/scales/biases, uint32 packed weights)."""
import numpy as np
import torch


def default_device():
    if not torch.cuda.is_available():
        raise RuntimeError("shardcompute_amd layers run on a GPU; none is visible")
    return torch.device("cuda", torch.cuda.current_device())


def to_device(a, device, dtype=None):
    """numpy / torch -> contiguous torch tensor on ``device`` (``dtype`` if given)."""
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        if a.dtype == np.uint32:
            t = torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).view(torch.uint32)
        elif a.dtype == np.uint16 and dtype == torch.bfloat16:
            # raw bf16 bit patterns
            t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
        else:
            t = torch.from_numpy(np.ascontiguousarray(a))
    elif isinstance(a, torch.Tensor):
        t = a
    else:
        t = torch.as_tensor(a)
    if dtype is not None and t.dtype != dtype:
        if dtype == torch.uint32 and t.dtype == torch.int32:
            t = t.view(torch.uint32)
        else:
            t = t.to(dtype)
    return t.to(device).contiguous()


def packed(a, device):
    """Packed MLX weights as uint32 on device (int32 bit patterns accepted)."""
    t = to_device(a, device)
    if t.dtype == torch.int32:
        t = t.view(torch.uint32)
    if t.dtype != torch.uint32:
        raise TypeError(f"quantized weights must be uint32, got {t.dtype}")
    return t


def nbytes(t):
    return 0 if t is None else t.numel() * t.element_size()
