"""Forward launcher: ``attention_forward`` returning (out, lse).

Mirrors the reference's ``attention_forward`` (kotflash/kernels/
triton_forward.py:372-456): outputs are allocated with torch (``out`` in the
input dtype, ``lse`` fp32 [B, Hq, Sq]); a non-causal short-query/long-key
problem takes the split-KV decode kernel with an LSE merge, everything else the
MFMA online-softmax forward.
"""
from __future__ import annotations

import torch

from .. import _hip
from .._planning import gfx950_decode_eligible, gfx950_head_dim_ok
from ._layout import padded_head_dim, prepare, require_hip_tensors, unpad


def hip_available() -> bool:
    """True when the HIP library loads and the current device is gfx950."""
    if not torch.cuda.is_available() or not _hip.library_available():
        return False
    return _hip.is_gfx950(torch.device("cuda", torch.cuda.current_device()))


def triton_available() -> bool:
    """Kept for import compatibility with the reference API: this build has no
    Triton kernels."""
    return False


def triton_turing_supported() -> bool:
    """Kept for import compatibility: always False (no Triton, no SM75)."""
    return False


def _check_shapes(q, k, v) -> None:
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("Expected q/k/v in [batch, heads, sequence, head_dim] layout")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[3] != k.shape[3]:
        raise ValueError("incompatible q/k/v shapes")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads (GQA/MQA)")
    if not gfx950_head_dim_ok(q.shape[3]):
        raise ValueError("HIP backend supports 8 <= head_dim <= 128")


def check_tuning_kwargs(block_m: int, block_n: int, num_warps: int, num_stages: int) -> None:
    """The reference launchers' tile-tuning keywords (triton_forward.py:
    372-376, triton_backward.py:335-339) are accepted so that drop-in callers
    such as its tile tuner keep working, and validated with the reference's
    messages (triton_forward.py:392-395). They select nothing here: the gfx950
    kernels' tiles are fixed per head dim by the MFMA, LDS and register plans."""
    if block_m <= 0 or block_n <= 0:
        raise ValueError("block_m and block_n must be positive")
    if num_warps <= 0 or num_stages <= 0:
        raise ValueError("num_warps and num_stages must be positive")


def attention_forward(q, k, v, *, causal: bool, scale: float, block_m: int = 64,
                      block_n: int = 32, num_warps: int = 4, num_stages: int = 2):
    """Run the HIP forward; returns ``(out, lse)``. The tuning keywords are
    the reference's (checked, otherwise unused)."""
    check_tuning_kwargs(block_m, block_n, num_warps, num_stages)
    require_hip_tensors("HIP attention forward", q, k, v)
    _check_shapes(q, k, v)
    return forward_validated(q, k, v, causal=causal, scale=scale)


def forward_validated(q, k, v, *, causal: bool, scale: float):
    """``attention_forward`` for callers that have already validated q/k/v as
    ``attention`` does (shapes, one device and dtype, and a HIP route: gfx950,
    fp16/bf16, 8 <= head_dim <= 128, the library loaded); it skips repeating
    those checks, which are a sizeable part of a small call's host time."""
    d = q.shape[3]
    dp = padded_head_dim(d)
    if dp == d and _hip.layout_ok(q) and _hip.layout_ok(k) and _hip.layout_ok(v):
        q_, k_, v_ = q, k, v
    else:
        q_, k_, v_ = prepare(q, dp), prepare(k, dp), prepare(v, dp)
    b, hq, sq, _ = q_.shape
    hkv, sk = k_.shape[1], k_.shape[2]
    out = torch.empty((b, hq, sq, dp), device=q.device, dtype=q.dtype)
    lse = torch.empty((b, hq, sq), device=q.device, dtype=torch.float32)
    if gfx950_decode_eligible(sq, sk, dp, causal=causal):
        splits = _hip.decode_num_splits(b, hq, hkv, sq, sk, dp)
        nbytes = _hip.decode_workspace_bytes(b, hq, hkv, sq, dp, splits)
        ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8) if nbytes else None
        _hip.decode(q_, k_, v_, out, lse, None, scale=scale, num_splits=splits, workspace=ws)
    else:
        _hip.fwd(q_, k_, v_, out, lse, causal=causal, scale=scale)
    return unpad(out, d), lse
