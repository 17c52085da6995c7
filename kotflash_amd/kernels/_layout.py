"""Input preparation shared by the launchers: the HIP kernels need a unit
head_dim stride, 16-byte aligned rows and a head_dim that is a multiple of 8.
Tensors that already satisfy this are passed through untouched (no copy);
others are made contiguous, and a head_dim that is not a multiple of 8 is
zero-padded (zero columns change neither Q K^T nor the kept columns of P V)."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _hip


def padded_head_dim(d: int) -> int:
    return -(-d // 8) * 8


def prepare(t: torch.Tensor, dp: int) -> torch.Tensor:
    d = t.shape[-1]
    if dp != d:
        return F.pad(t, (0, dp - d)).contiguous()
    if not _hip.layout_ok(t):
        return t.contiguous()
    return t


def unpad(t: torch.Tensor, d: int) -> torch.Tensor:
    return t if t.shape[-1] == d else t[..., :d].contiguous()


def require_hip_tensors(what: str, *tensors: torch.Tensor) -> None:
    """Fail loudly (no fallback) when the HIP path cannot run these tensors."""
    # Plain loops: this runs on every decode call, where generator
    # expressions cost measurable host time.
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(f"{what} requires GPU tensors")
    dtype = tensors[0].dtype
    if dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"{what} supports float16 and bfloat16 only")
    for t in tensors:
        if t.dtype != dtype:
            raise TypeError(f"{what}: all tensors must share one dtype")
    dev = tensors[0].device
    for t in tensors:
        if t.device != dev:
            raise ValueError(f"{what}: all tensors must be on the same device")
    if not _hip.is_gfx950(dev):
        raise RuntimeError(f"{what} requires an AMD gfx950 (MI355X) device")
    _hip.lib()  # raises RuntimeError when the library is missing
