"""The HIP kernels as ``torch.library`` custom operators.

The reference wraps its Triton launchers in a ``torch.autograd.Function``
(kotflash/attention.py:203-220). Here the same launchers are registered as
custom ops in the ``kotflash_amd`` namespace, each with a fake (shape-only)
implementation and, for attention, a registered backward:

- ``kotflash_amd::attn_fwd(q, k, v, causal, scale) -> (out, lse)``
- ``kotflash_amd::attn_bwd(q, k, v, out, lse, grad_out, causal, scale) -> (dq, dk, dv)``
- ``kotflash_amd::decode(q, k, v, scale) -> out`` (split-KV decode over
  K/V views read in place, inference only)
- ``kotflash_amd::kv_append_(k_cache, v_cache, new_k, new_v, start) -> ()``
  (mutates both caches)
- ``kotflash_amd::append_decode_(q, k_cache, v_cache, new_k, new_v,
  past_length, scale) -> out`` (fused one-token append + split-KV decode,
  reference kotflash/kernels/triton_decode.py:302-386; mutates both caches)

``torch.compile`` traces through them without graph breaks: the fake
implementations give it output shapes, dtypes and strides, and autograd
differentiates ``attn_fwd`` through ``attn_bwd``. Outputs are always
fresh contiguous tensors, as the fake implementations state.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .kernels.hip_backward import attention_backward
from .kernels.hip_decode import attention_forward_strided_append, attention_forward_strided_decode
from .kernels.hip_forward import attention_forward

__all__ = ["attn_fwd", "attn_bwd", "decode", "kv_append_", "append_decode_"]


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


@torch.library.custom_op("kotflash_amd::attn_fwd", mutates_args=())
def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
             scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention forward (O in q's dtype, natural-log LSE in fp32)."""
    out, lse = attention_forward(q, k, v, causal=causal, scale=scale)
    return _contig(out), lse


@attn_fwd.register_fake
def _attn_fwd_fake(q, k, v, causal, scale):
    b, hq, sq, d = q.shape
    out = q.new_empty((b, hq, sq, d))
    lse = q.new_empty((b, hq, sq), dtype=torch.float32)
    return out, lse


@torch.library.custom_op("kotflash_amd::attn_bwd", mutates_args=())
def attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
             lse: torch.Tensor, grad_out: torch.Tensor, causal: bool,
             scale: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Attention backward: (dQ, dK, dV) in the inputs' dtypes, dK/dV summed
    over each GQA group."""
    dq, dk, dv = attention_backward(q, k, v, out, lse, grad_out, causal=causal, scale=scale)
    return _contig(dq), _contig(dk), _contig(dv)


@attn_bwd.register_fake
def _attn_bwd_fake(q, k, v, out, lse, grad_out, causal, scale):
    return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape)


def _attn_setup_context(ctx, inputs, output):
    q, k, v, causal, scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse)
    ctx.causal = causal
    ctx.scale = scale
    ctx.mark_non_differentiable(lse)


def _attn_backward(ctx, grad_out, grad_lse):
    q, k, v, out, lse = ctx.saved_tensors
    dq, dk, dv = attn_bwd(q, k, v, out, lse, _contig(grad_out), ctx.causal, ctx.scale)
    return dq, dk, dv, None, None


attn_fwd.register_autograd(_attn_backward, setup_context=_attn_setup_context)


@torch.library.custom_op("kotflash_amd::decode", mutates_args=())
def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Split-KV decode (short non-causal query block against long K/V views);
    returns O."""
    return _contig(attention_forward_strided_decode(q, k, v, scale=scale))


@decode.register_fake
def _decode_fake(q, k, v, scale):
    return q.new_empty(q.shape)


@torch.library.custom_op("kotflash_amd::kv_append_", mutates_args=("k_cache", "v_cache"))
def kv_append_(k_cache: torch.Tensor, v_cache: torch.Tensor, new_k: torch.Tensor,
               new_v: torch.Tensor, start: int) -> None:
    """cache[:, :, start:start + n] = new for K and V (the reference's
    ``append_kv_`` pybind op, kotflash/csrc/kv_append.cpp:4-14, with its
    checks: matching 4-D shapes, fp16/bf16, unit head_dim stride, capacity)."""
    from . import _hip
    from .cache import _validate_kv_tensors
    from .kernels._layout import require_hip_tensors

    _validate_kv_tensors(k_cache, v_cache, new_k, new_v)
    require_hip_tensors("kv_append_", k_cache, v_cache, new_k, new_v)
    if k_cache.stride(3) != 1 or v_cache.stride(3) != 1:
        raise ValueError("K/V caches need a unit head_dim stride")
    if start < 0 or start + new_k.shape[2] > k_cache.shape[2]:
        raise ValueError("KV cache capacity exceeded")
    _hip.kv_append(k_cache, v_cache, new_k, new_v, start=start)


@kv_append_.register_fake
def _kv_append_fake(k_cache, v_cache, new_k, new_v, start):
    return None


@torch.library.custom_op("kotflash_amd::append_decode_", mutates_args=("k_cache", "v_cache"))
def append_decode_(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   new_k: torch.Tensor, new_v: torch.Tensor, past_length: int,
                   scale: float) -> torch.Tensor:
    """Store one new token at ``past_length`` of both caches and attend with
    q [B, Hq, 1, D] over the first past_length + 1 positions (the split kernel
    writes the token; two launches). Returns O."""
    return _contig(attention_forward_strided_append(q, k_cache, v_cache, new_k, new_v,
                                                    past_length=past_length, scale=scale))


@append_decode_.register_fake
def _append_decode_fake(q, k_cache, v_cache, new_k, new_v, past_length, scale):
    return q.new_empty(q.shape)
