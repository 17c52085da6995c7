"""Public attention API: validation, routing, SDPA path and the HIP autograd op.

Drop-in for the reference's ``kotflash.attention`` (kotflash/attention.py
:1-312): same signature, validation order and messages, default scale,
upper-left causal mask, MHA/GQA/MQA mapping and SDPA fallback. The custom
kernel backend is ``"hip"``; ``"triton"`` is accepted as an alias with the
same fail-loudly semantics, so callers written against the reference keep
working. On MI355X (gfx950), ``"auto"`` routes fp16/bf16 problems with
8 <= head_dim <= 128 to the HIP kernels; everything else uses SDPA.
"""
from __future__ import annotations

import math
from functools import lru_cache
from typing import Optional

import torch
import torch.nn.functional as F

from . import _hip
from ._planning import gfx950_profile_for_shapes, t4_profile_for_shapes
from .kernels.hip_backward import attention_backward, backward_validated
from .kernels.hip_decode import (  # noqa: F401  strided_decode_supported: the reference's module name
    decode_supported_unchecked,
    strided_decode_supported,
    validated_decode_supported,
)
from .kernels.hip_forward import attention_forward, forward_validated, triton_turing_supported

BACKENDS = ("auto", "hip", "triton", "sdpa")
_DTYPE_NAMES = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Input contract of the reference (kotflash/attention.py:21-45), in the
    same order and with the same messages."""
    if not (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor)
            and isinstance(v, torch.Tensor)):
        raise TypeError("q, k and v must be torch.Tensor instances")
    qs, ks, vs = q.shape, k.shape, v.shape
    if len(qs) != 4 or len(ks) != 4 or len(vs) != 4:
        raise ValueError("Expected q/k/v in [batch, heads, sequence, head_dim] layout")
    if qs[0] == 0:
        raise ValueError("Batch dimension must be non-zero")
    if qs[1] == 0 or ks[1] == 0:
        raise ValueError("Head dimensions must be non-zero")
    if qs[3] == 0:
        raise ValueError("Head dimension must be non-zero")
    if qs[0] != ks[0] or qs[0] != vs[0]:
        raise ValueError("Batch dimensions must match")
    if ks != vs:
        raise ValueError("K and V shapes must match")
    if qs[3] != ks[3]:
        raise ValueError("Q/K/V head dimensions must match")
    if qs[1] % ks[1] != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads (GQA/MQA)")
    dev = q.device
    if dev != k.device or dev != v.device:
        raise ValueError("Q/K/V must be on the same device")
    dt = q.dtype
    if dt != k.dtype or dt != v.dtype:
        raise ValueError("Q/K/V dtypes must match")
    if qs[2] == 0 or ks[2] == 0:
        raise ValueError("Sequence dimensions must be non-zero")


def _sdpa_kwargs(q, *, causal: bool, scale: Optional[float]):
    """SDPA keyword arguments. A scale equal to the default 1/sqrt(D) (within
    1e-12) is left out so PyTorch keeps its default-scale dispatch (reference
    kotflash/attention.py:48-61)."""
    kwargs = {"attn_mask": None, "dropout_p": 0.0, "is_causal": causal}
    if scale is not None:
        default = 1.0 / math.sqrt(q.shape[-1])
        if not math.isclose(scale, default, rel_tol=0.0, abs_tol=1e-12):
            kwargs["scale"] = scale
    return kwargs


def _sdpa_expanded(q, k, v, *, causal: bool, scale: Optional[float]):
    """SDPA on K/V heads repeated to Hq (reference kotflash/attention.py:64-71)."""
    group = q.shape[1] // k.shape[1]
    if group != 1:
        k = k.repeat_interleave(group, dim=1)
        v = v.repeat_interleave(group, dim=1)
    return F.scaled_dot_product_attention(q, k, v, **_sdpa_kwargs(q, causal=causal, scale=scale))


def _sdpa(q, k, v, *, causal: bool, scale: Optional[float]):
    """SDPA with native GQA; repeats K/V only when this PyTorch has no
    ``enable_gqa`` (reference kotflash/attention.py:120-135)."""
    kwargs = _sdpa_kwargs(q, causal=causal, scale=scale)
    if q.shape[1] != k.shape[1]:
        try:
            return F.scaled_dot_product_attention(q, k, v, enable_gqa=True, **kwargs)
        except TypeError as exc:
            if "enable_gqa" not in str(exc):
                raise
            return _sdpa_expanded(q, k, v, causal=causal, scale=scale)
    return F.scaled_dot_product_attention(q, k, v, **kwargs)


@lru_cache(maxsize=8)
def _is_measured_t4_runtime(device_index: int) -> bool:
    """The reference's exact-stack T4 gate (kotflash/attention.py:74-87). It
    requires CUDA 12.4 on a Tesla T4, so it is False on every ROCm stack. The
    conditions that need no device query are tested first."""
    if not triton_turing_supported() or torch.version.cuda != "12.4":
        return False
    device = torch.device("cuda", device_index)
    return (
        torch.cuda.is_available()
        and torch.cuda.get_device_capability(device) == (7, 5)
        and torch.cuda.get_device_name(device) == "Tesla T4"
        and torch.__version__.split("+", 1)[0] == "2.6.0"
    )


def _device_index(t: torch.Tensor) -> int:
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _t4_profile_backend(q, k, v, *, causal: bool, scale: float):
    """Backend for an exact measured T4 shape (reference attention.py:90-106)."""
    if not q.is_cuda or q.dtype != torch.float16:
        return None
    if not triton_turing_supported() or not _is_measured_t4_runtime(_device_index(q)):
        return None
    return t4_profile_for_shapes(
        tuple(q.shape), tuple(k.shape), tuple(v.shape), causal=causal, scale=scale,
        contiguous=q.is_contiguous() and k.is_contiguous() and v.is_contiguous(),
    )


def _gfx950_profile_backend(q, k, v, *, causal: bool, needs_grad: bool = True):
    """``"hip"`` when ``auto`` should use the HIP kernels on this device."""
    if not q.is_cuda or not _hip.is_gfx950(q.device):
        return None
    route = gfx950_profile_for_shapes(
        q.shape, k.shape, causal=causal, dtype_name=_DTYPE_NAMES.get(q.dtype, ""),
        needs_grad=needs_grad,
    )
    if route == "hip" and not _hip.library_available():
        # A gfx950 device without the library is a broken install, not an
        # unsupported shape: fail loudly instead of silently running SDPA.
        _hip.lib()
    return route


def _blockwise_backward(q, k, v, out, lse, grad_out, *, causal: bool, scale: float,
                        q_block: int = 64, kv_block: int = 128):
    """Memory-bounded fp32 backward in plain PyTorch (tile recomputation, GQA
    group sum), kept as the reference keeps it (kotflash/attention.py:138-201):
    a utility for tests, not used by ``attention``."""
    bsz, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    group = hq // hkv
    qf, kf, vf, of, gf = (t.float() for t in (q, k, v, out, grad_out))
    lsef = lse.float()
    dq = torch.zeros_like(qf)
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    for q0 in range(0, sq, q_block):
        q1 = min(q0 + q_block, sq)
        qb, gb, lb = qf[:, :, q0:q1], gf[:, :, q0:q1], lsef[:, :, q0:q1]
        delta = (of[:, :, q0:q1] * gb).sum(-1, keepdim=True)
        rows = torch.arange(q0, q1, device=q.device)
        for k0 in range(0, sk, kv_block):
            k1 = min(k0 + kv_block, sk)
            kb = kf[:, :, k0:k1].repeat_interleave(group, dim=1)
            vb = vf[:, :, k0:k1].repeat_interleave(group, dim=1)
            s = torch.matmul(qb, kb.transpose(-2, -1)) * scale
            if causal:
                cols = torch.arange(k0, k1, device=q.device)
                s = s.masked_fill(cols[None, :] > rows[:, None], float("-inf"))
            p = torch.nan_to_num(torch.exp(s - lb[..., None]), nan=0.0, posinf=0.0, neginf=0.0)
            ds = p * (torch.matmul(gb, vb.transpose(-2, -1)) - delta)
            dq[:, :, q0:q1] += torch.matmul(ds, kb) * scale
            dkg = torch.matmul(ds.transpose(-2, -1), qb) * scale
            dvg = torch.matmul(p.transpose(-2, -1), gb)
            dk[:, :, k0:k1] += dkg.reshape(bsz, hkv, group, k1 - k0, d).sum(2)
            dv[:, :, k0:k1] += dvg.reshape(bsz, hkv, group, k1 - k0, d).sum(2)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


class _HipAttention(torch.autograd.Function):
    """Eager autograd over the HIP forward/backward; saves (q, k, v, out, lse)
    as the reference's custom op does (kotflash/attention.py:203-220)."""

    @staticmethod
    def forward(ctx, q, k, v, causal: bool, scale: float):
        out, lse = forward_validated(q, k, v, causal=causal, scale=scale)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal = causal
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse = ctx.saved_tensors
        if grad_out.shape != out.shape or grad_out.dtype != out.dtype or grad_out.device != out.device:
            dq, dk, dv = attention_backward(
                q, k, v, out, lse, grad_out, causal=ctx.causal, scale=ctx.scale
            )
        else:
            dq, dk, dv = backward_validated(
                q, k, v, out, lse, grad_out, causal=ctx.causal, scale=ctx.scale
            )
        return dq, dk, dv, None, None


def _hip_op_attention(q, k, v, causal: bool, scale: float) -> torch.Tensor:
    """O from the HIP kernels. Under torch.compile: the
    ``kotflash_amd::attn_fwd`` custom op, whose registered backward is
    ``kotflash_amd::attn_bwd``. In eager mode the same launchers are called
    through ``_HipAttention`` (gradients needed) or directly (inference),
    which costs less host time than the op's dispatch: about 70 us less per
    training step at config 1."""
    if torch.compiler.is_compiling():
        from .ops import attn_fwd

        return attn_fwd(q, k, v, causal, scale)[0]
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        out = _HipAttention.apply(q, k, v, causal, scale)
    else:
        out = forward_validated(q, k, v, causal=causal, scale=scale)[0]
    return out if out.is_contiguous() else out.contiguous()


def hip_supported(q: torch.Tensor, k: torch.Tensor) -> bool:
    """Whether the explicit HIP backend can run this problem."""
    return (
        q.is_cuda
        and q.dtype in (torch.float16, torch.bfloat16)
        and 8 <= q.shape[-1] <= 128
        and _hip.is_gfx950(q.device)
        and _hip.library_available()
    )


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool = False,
    scale: Optional[float] = None,
    backend: str = "auto",
) -> torch.Tensor:
    """Scaled dot-product attention with MHA, GQA and MQA support.

    Tensors use [batch, heads, sequence, head_dim]; Hq must be divisible by
    Hkv (query head h uses KV head h // (Hq / Hkv)). The causal mask is
    upper-left aligned (key j visible to query i iff j <= i), as in PyTorch
    SDPA.

    backend is one of auto, hip, triton (alias of hip) or sdpa. hip needs an
    MI355X (gfx950) GPU, fp16 or bf16 and 8 <= head_dim <= 128, and raises
    RuntimeError otherwise. For non-causal short queries (Sq <= 16) against
    long caches (Sk >= 1024) without autograd, the HIP path reads K/V in place
    (padded ``PreallocatedKVCache`` views included) with split-KV decode; the
    caller must pass only keys visible to every query. On gfx950, auto uses
    the HIP kernels for fp16/bf16 inference calls and decode shapes, and for
    training calls (autograd) of at least 1.5e9 forward FLOP, below which an
    eager training step is host-bound and SDPA finishes first; SDPA
    everywhere else.
    """
    _validate(q, k, v)
    if not isinstance(causal, bool):
        raise TypeError("causal must be a bool")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    else:
        try:
            scale = float(scale)
        except (TypeError, ValueError) as exc:
            raise TypeError("scale must be a finite real number or None") from exc
        if not math.isfinite(scale):
            raise ValueError("scale must be finite")
    if backend not in BACKENDS:
        raise ValueError("backend must be one of: auto, hip, triton, sdpa")

    explicit = backend in ("hip", "triton")
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad
                                              or v.requires_grad)
    route = None
    if backend == "auto":
        route = _gfx950_profile_backend(q, k, v, causal=causal, needs_grad=needs_grad)

    # Inference on preallocated caches: read the (padded) K/V views in place.
    if (explicit or route == "hip") and not causal and not needs_grad \
            and validated_decode_supported(q, k, v):
        return decode_supported_unchecked(q, k, v, float(scale))

    if explicit:
        if not hip_supported(q, k):
            raise RuntimeError(
                "HIP backend requires an AMD MI355X (gfx950) GPU with the kotflash_amd "
                "library built, FP16 or BF16 and 8 <= head_dim <= 128"
            )
        return _hip_op_attention(q, k, v, causal, float(scale))

    if backend == "auto":
        if route == "hip":
            return _hip_op_attention(q, k, v, causal, float(scale))
        profile = _t4_profile_backend(q, k, v, causal=causal, scale=float(scale))
        if profile == "sdpa_expanded":
            return _sdpa_expanded(q, k, v, causal=causal, scale=scale)

    # Conservative fallback for other devices, dtypes and shapes.
    return _sdpa(q, k, v, causal=causal, scale=scale)
