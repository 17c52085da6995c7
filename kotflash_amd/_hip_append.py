"""One-launch K/V cache append on gfx950.

Counterpart of the reference's optional CUDA op (kotflash/_cuda_append.py:31-44
and kotflash/csrc/kv_append_cuda.cu:50-75): same argument checks, same
exceptions, but the library is built ahead of time (no JIT), fp16 and bf16 are
accepted, and ``start`` may be a per-sequence device tensor.
"""
from __future__ import annotations

from typing import Optional, Sequence, Union

import torch

from . import _hip


def append_kv_hip(k_cache, v_cache, new_k, new_v, start: Union[int, torch.Tensor], *,
                  host_starts: Optional[Sequence[int]] = None) -> None:
    """Write new_k/new_v [B, H, S, D] into the caches [B, H, capacity, D] at
    positions start .. start+S-1 (``start`` an int, or a device int64 [B]
    tensor of per-sequence positions).

    Every position is range-checked before anything is written, as the
    reference's op does (kv_append_cuda.cu:50-75): an append that would leave
    [0, capacity) raises RuntimeError and the caches stay unchanged. For a
    device ``start`` tensor the check uses ``host_starts`` (the same positions
    on the host, e.g. a cache's own length mirror) when given, and otherwise
    copies ``start`` to the host, which synchronizes with the device."""
    # Written out check by check: this runs on every decode step, and
    # generator expressions over the four tensors cost microseconds of host time.
    if not (k_cache.is_cuda and v_cache.is_cuda and new_k.is_cuda and new_v.is_cuda):
        raise ValueError("all cache and source tensors must be GPU tensors")
    dtype, ok = k_cache.dtype, (torch.float16, torch.bfloat16)
    if (dtype not in ok or v_cache.dtype not in ok or new_k.dtype not in ok
            or new_v.dtype not in ok):
        raise TypeError("the HIP append kernel supports FP16 and BF16 only")
    if v_cache.dtype != dtype or new_k.dtype != dtype or new_v.dtype != dtype:
        raise TypeError("all cache and source tensors must share one dtype")
    dev = k_cache.device
    if v_cache.device != dev or new_k.device != dev or new_v.device != dev:
        raise ValueError("all cache and source tensors must be on the same GPU")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise RuntimeError("K/V cache must have matching [B,H,capacity,D] shapes")
    if new_k.dim() != 4 or new_v.shape != new_k.shape:
        raise RuntimeError("new K/V must have matching [B,H,S,D] shapes")
    if k_cache.stride(3) != 1 or v_cache.stride(3) != 1:
        raise RuntimeError("destination K/V caches need a unit head_dim stride")
    if (new_k.shape[0] != k_cache.shape[0] or new_k.shape[1] != k_cache.shape[1]
            or new_k.shape[3] != k_cache.shape[3]):
        raise RuntimeError("new K/V batch, heads and head_dim must match the cache")
    if new_k.shape[2] <= 0 or new_k.shape[3] <= 0:
        raise RuntimeError("new K/V dimensions must be non-empty")
    if not _hip.is_gfx950(k_cache.device):
        raise RuntimeError("the HIP append kernel requires an AMD gfx950 (MI355X) device")
    if isinstance(start, torch.Tensor):
        if start.dtype != torch.int64 or start.device != k_cache.device or start.shape != (new_k.shape[0],):
            raise ValueError("per-sequence start must be a device int64 tensor of shape [B]")
        # The kernel reads start[b] as a dense array: an expanded or strided
        # view is materialised first.
        if not start.is_contiguous():
            start = start.contiguous()
        starts = start.tolist() if host_starts is None else host_starts
        if len(starts) != new_k.shape[0]:
            raise ValueError("host_starts must have one entry per batch element")
        n, capacity = new_k.shape[2], k_cache.shape[2]
        for s in starts:
            if s < 0 or s + n > capacity:
                raise RuntimeError("append range exceeds cache capacity")
        _hip.kv_append(k_cache, v_cache, new_k, new_v, start_dev=start, max_start=max(starts))
    else:
        start = int(start)
        if start < 0 or start + new_k.shape[2] > k_cache.shape[2]:
            raise RuntimeError("append range exceeds cache capacity")
        _hip.kv_append(k_cache, v_cache, new_k, new_v, start=start)


# Name kept for drop-in callers of the reference's op.
append_kv_cuda = append_kv_hip
