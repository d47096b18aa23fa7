"""GPU-side helpers for tests and bench (torch is only device memory here)."""
from __future__ import annotations

import numpy as np


def to_dev(torch, bits: np.ndarray, stride0: int | None = None):
    """uint16 bf16 bits [R, C] -> CUDA bfloat16 tensor (optionally row-padded)."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    if stride0 is not None and stride0 != bits.shape[1]:
        pad = np.zeros((bits.shape[0], stride0), np.uint16)
        pad[:, :bits.shape[1]] = bits
        t = torch.from_numpy(pad.view(np.int16)).view(torch.bfloat16).cuda()
        return t[:, :bits.shape[1]]
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()


def from_dev(t) -> np.ndarray:
    """CUDA tensor -> numpy (bf16 as uint16 bits, fp32 as float32)."""
    import torch
    if t.dtype == torch.bfloat16:
        return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().cpu().numpy()
