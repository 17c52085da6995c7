"""Backward launcher: ``attention_backward`` returning (dq, dk, dv).

Mirrors the reference's ``attention_backward`` (kotflash/kernels/
triton_backward.py:335-421): gradients are allocated with torch in the input
dtypes, dK/dV are summed over each GQA group, and the row delta is computed
from the stored low-precision O. The workspace (fp32 row deltas) comes from
torch's caching allocator.
"""
from __future__ import annotations

import torch

from .. import _hip
from ._layout import padded_head_dim, prepare, require_hip_tensors, unpad
from .hip_forward import _check_shapes, check_tuning_kwargs


def attention_backward(q, k, v, out, lse, grad_out, *, causal: bool, scale: float,
                       block_m: int = 32, block_n: int = 64, num_warps: int = 4,
                       num_stages: int = 1):
    """Run the HIP backward; returns ``(dq, dk, dv)``. The tuning keywords are
    the reference's (checked, otherwise unused)."""
    check_tuning_kwargs(block_m, block_n, num_warps, num_stages)
    require_hip_tensors("HIP attention backward", q, k, v, out, grad_out)
    _check_shapes(q, k, v)
    if out.shape != q.shape or grad_out.shape != q.shape:
        raise ValueError("out and grad_out must have q's shape")
    if lse.shape != q.shape[:3] or lse.dtype != torch.float32:
        raise ValueError("lse must be float32 [B, Hq, Sq]")
    return backward_validated(q, k, v, out, lse, grad_out, causal=causal, scale=scale)


def backward_validated(q, k, v, out, lse, grad_out, *, causal: bool, scale: float):
    """``attention_backward`` for the autograd path, whose q/k/v/out/lse come
    from a validated HIP forward and whose grad_out autograd gives out's
    shape and dtype: it skips repeating those checks (a small step's host
    time). grad_out's layout is still prepared like every other input."""
    d = q.shape[3]
    dp = padded_head_dim(d)
    q_, k_, v_, o_, do_ = (prepare(t, dp) for t in (q, k, v, out, grad_out))
    lse_ = lse.contiguous()
    b, hq, sq, _ = q_.shape
    hkv, sk = k_.shape[1], k_.shape[2]
    dq = torch.empty_like(q_, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k_, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v_, memory_format=torch.contiguous_format)
    nbytes = _hip.bwd_workspace_bytes(b, hq, hkv, sq, sk, dp, causal)
    ws = torch.empty(max(nbytes, 256), device=q.device, dtype=torch.uint8)
    _hip.bwd(q_, k_, v_, o_, lse_, do_, dq, dk, dv, causal=causal, scale=scale, workspace=ws)
    return unpad(dq, d), unpad(dk, d), unpad(dv, d)
