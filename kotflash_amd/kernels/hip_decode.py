"""Decode launchers for preallocated (possibly padded) K/V caches.

Mirrors the reference's stride-aware decode module (kotflash/kernels/
triton_decode.py:302-468): ``strided_decode_supported``,
``attention_forward_strided_decode`` and ``attention_forward_strided_append``,
plus ``attention_decode_ragged`` for caches whose sequences have different
lengths (one launch for all of them, keys beyond each sequence's length
masked).
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from .. import _hip
from .._planning import GFX950_DECODE_MAX_SQ, GFX950_DECODE_MIN_SK, gfx950_head_dim_ok
from ._layout import padded_head_dim, prepare, require_hip_tensors


def strided_decode_supported(q, k, v) -> bool:
    """Whether the HIP split-KV decode reads these tensors in place: GPU
    fp16/bf16 on gfx950, a short query (Sq <= 16) against a long key sequence
    (Sk >= 1024), 8 <= D <= 128 with D a multiple of 8, and layouts with a unit
    head_dim stride, 8-element multiple strides and 16-byte alignment -- which
    includes the padded prefix views of ``PreallocatedKVCache`` (reference
    triton_decode.py:389-409 accepts only D <= 64 and fp16)."""
    if not (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor)
            and isinstance(v, torch.Tensor)):
        return False
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    qs, ks = q.shape, k.shape
    if len(qs) != 4 or len(ks) != 4 or v.shape != ks:
        return False
    if qs[0] != ks[0] or qs[1] % ks[1] or qs[3] != ks[3]:
        return False
    d = qs[3]
    if qs[2] > GFX950_DECODE_MAX_SQ or ks[2] < GFX950_DECODE_MIN_SK:
        return False
    if not gfx950_head_dim_ok(d) or d % 8:
        return False
    if not (_hip.layout_ok(q) and _hip.layout_ok(k) and _hip.layout_ok(v)):
        return False
    return _hip.is_gfx950(q.device) and _hip.library_available()


_DECODE_DTYPES = (torch.float16, torch.bfloat16)


def validated_decode_supported(q, k, v) -> bool:
    """``strided_decode_supported`` for inputs that already passed the public
    ``attention``'s validation (tensors, 4-D, matching batch and head_dim,
    head grouping, one device, one dtype): only the decode envelope, the
    layouts and the device remain to check."""
    if not q.is_cuda or q.dtype not in _DECODE_DTYPES:
        return False
    qs, ks = q.shape, k.shape
    if qs[2] > GFX950_DECODE_MAX_SQ or ks[2] < GFX950_DECODE_MIN_SK:
        return False
    d = qs[3]
    if d % 8 or not gfx950_head_dim_ok(d):
        return False
    if not (_hip.layout_ok(q) and _hip.layout_ok(k) and _hip.layout_ok(v)):
        return False
    return _hip.is_gfx950(q.device) and _hip.library_available()


def _decode(q, k, v, seqlens: Optional[torch.Tensor], scale: float, with_lse: bool,
            host_lengths: Optional[Sequence[int]] = None):
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    out = torch.empty((b, hq, sq, d), device=q.device, dtype=q.dtype)
    lse = torch.empty((b, hq, sq), device=q.device, dtype=torch.float32) if with_lse else None
    if host_lengths is not None and max(host_lengths) == sk:
        splits = _hip.decode_num_splits_ragged(b, hq, hkv, sq, host_lengths, d)
    else:
        splits = _hip.decode_num_splits(b, hq, hkv, sq, sk, d)
    nbytes = _hip.decode_workspace_bytes(b, hq, hkv, sq, d, splits)
    ws = _hip.workspace(q.device, nbytes) if nbytes else None
    _hip.decode(q, k, v, out, lse, seqlens, scale=scale, num_splits=splits, workspace=ws)
    return out, lse


def attention_forward_strided_decode(q, k, v, *, scale: float):
    """Inference-only split-KV decode reading (padded) K/V views in place;
    returns O (reference triton_decode.py:412-468)."""
    if not strided_decode_supported(q, k, v):
        raise ValueError(
            "expected fp16/bf16 gfx950 tensors with a short query, a long key "
            "sequence and an inner-contiguous, 16-byte aligned K/V layout"
        )
    return _decode(q, k, v, None, float(scale), with_lse=False)[0]


def decode_supported_unchecked(q, k, v, scale: float):
    """``attention_forward_strided_decode`` for a caller that has just
    checked ``validated_decode_supported(q, k, v)`` (the public
    ``attention``), without checking again."""
    return _decode(q, k, v, None, float(scale), with_lse=False)[0]


def attention_forward_strided_append(q, k_cache, v_cache, new_k, new_v, *,
                                     past_length: int, scale: float):
    """Append one token at ``past_length`` and attend over the first
    ``past_length + 1`` cache positions; returns O.

    Same contract as the reference (triton_decode.py:302-386): two launches,
    a split kernel that also writes the slot and the LSE merge. The split
    kernel's last split attends to the new token straight from ``new_k`` /
    ``new_v`` and stores it into the cache (``kf_attn_append_decode``); the
    other splits read positions [0, past_length) in place. Head dims that are
    not a multiple of 8 take a separate append launch and a padded decode.
    """
    require_hip_tensors("fused append/decode", q, k_cache, v_cache, new_k, new_v)
    if q.ndim != 4 or q.shape[2] != 1:
        raise ValueError("q must be [B,Hq,1,D]")
    if k_cache.ndim != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("K/V cache must have matching [B,Hkv,capacity,D] shapes")
    if k_cache.stride(3) != 1 or v_cache.stride(3) != 1:
        raise ValueError("destination K/V cache buffers need a unit head_dim stride")
    if new_k.ndim != 4 or new_v.shape != new_k.shape or new_k.shape[2] != 1:
        raise ValueError("new K/V must have matching [B,Hkv,1,D] shapes")
    b, hq, _, d = q.shape
    _, hkv, capacity, cache_d = k_cache.shape
    if cache_d != d or new_k.shape != (b, hkv, 1, d):
        raise ValueError("query, cache and new K/V shapes are incompatible")
    if hq % hkv or past_length < 0 or past_length + 1 > capacity:
        raise ValueError("unsupported head grouping, cache length or capacity")
    # The fused kernel addresses the whole cache (its store may land anywhere
    # below the capacity) with 32-bit buffer offsets; the two-launch path
    # only needs the visible prefix to fit.
    fits = (((capacity - 1) * k_cache.stride(2) + d) * 2 < 2 ** 31
            and ((capacity - 1) * v_cache.stride(2) + d) * 2 < 2 ** 31)
    if (d % 8 == 0 and fits and _hip.layout_ok(q) and _hip.layout_ok(k_cache)
            and _hip.layout_ok(v_cache)):
        if not _hip.layout_ok(new_k):
            new_k = new_k.contiguous()
        if not _hip.layout_ok(new_v):
            new_v = new_v.contiguous()
        return _append_decode(q, k_cache, v_cache, new_k, new_v, None, past_length,
                              past_length, float(scale), with_lse=False)[0]
    _hip.kv_append(k_cache, v_cache, new_k, new_v, start=past_length)
    k_view = k_cache[:, :, : past_length + 1]
    v_view = v_cache[:, :, : past_length + 1]
    dp = padded_head_dim(d)
    if dp != d or not all(_hip.layout_ok(t) for t in (q, k_view, v_view)):
        q, k_view, v_view = (prepare(t, dp) for t in (q, k_view, v_view))
    out = _decode(q, k_view, v_view, None, float(scale), with_lse=False)[0]
    return out[..., :d].contiguous() if dp != d else out


def _append_decode(q, k_cache, v_cache, new_k, new_v, lengths: Optional[torch.Tensor],
                   past_length: int, max_length: int, scale: float, with_lse: bool,
                   host_lengths: Optional[Sequence[int]] = None):
    b, hq, sq, d = q.shape
    hkv = k_cache.shape[1]
    out = torch.empty((b, hq, sq, d), device=q.device, dtype=q.dtype)
    lse = torch.empty((b, hq, sq), device=q.device, dtype=torch.float32) if with_lse else None
    if host_lengths is not None and max_length > 0:
        splits = _hip.decode_num_splits_ragged(b, hq, hkv, sq, host_lengths, d)
    else:
        splits = _hip.decode_num_splits(b, hq, hkv, sq, max_length, d)
    nbytes = _hip.decode_workspace_bytes(b, hq, hkv, sq, d, splits + 1)
    ws = _hip.workspace(q.device, nbytes)
    _hip.append_decode(q, k_cache, v_cache, new_k, new_v, out, lse, lengths,
                       past_length=past_length, max_length=max_length, scale=scale,
                       num_splits=splits, workspace=ws)
    return out, lse


def attention_append_decode_ragged(q, k_cache, v_cache, new_k, new_v, seqlens: torch.Tensor, *,
                                   host_lengths: Sequence[int], scale: float,
                                   with_lse: bool = False):
    """Append new_k/new_v [B, Hkv, n, D] at each sequence's position
    ``seqlens[b]`` (device int32 [B], equal to ``host_lengths``) and run
    non-causal decode in which the rows of sequence b see its first
    seqlens[b] + n positions after the append: one decode launch and one
    merge (``kf_attn_append_decode``). Callers validate capacity first.
    Returns O, or (O, LSE) with ``with_lse``."""
    require_hip_tensors("ragged append/decode", q, k_cache, v_cache, new_k, new_v)
    if seqlens.dtype != torch.int32 or seqlens.device != q.device or seqlens.shape != (q.shape[0],):
        raise ValueError("seqlens must be a device int32 tensor of shape [B]")
    if not seqlens.is_contiguous():  # the kernel reads seqlens[b] as a dense array
        seqlens = seqlens.contiguous()
    if q.ndim != 4 or k_cache.ndim != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("expected [B,H,S,D] query and cache tensors")
    if new_k.ndim != 4 or new_v.shape != new_k.shape or new_k.shape[2] <= 0:
        raise ValueError("new K/V must have matching non-empty [B,Hkv,n,D] shapes")
    b, hq, _, d = q.shape
    _, hkv, capacity, _ = k_cache.shape
    if k_cache.shape[0] != b or hq % hkv or k_cache.shape[3] != d or new_k.shape[:2] != (b, hkv) \
            or new_k.shape[3] != d:
        raise ValueError("query, cache and new K/V shapes are incompatible")
    if d % 8 or not gfx950_head_dim_ok(d):
        raise ValueError("ragged append/decode needs head_dim a multiple of 8 in [8, 128]")
    host_lengths = [int(x) for x in host_lengths]
    if len(host_lengths) != b:
        raise ValueError("host_lengths must have one entry per batch element")
    if min(host_lengths) < 0 or max(host_lengths) + new_k.shape[2] > capacity:
        raise ValueError("appended tokens must fit the cache capacity")
    if not all(_hip.layout_ok(t) for t in (q, k_cache, v_cache)):
        raise ValueError("ragged append/decode needs inner-contiguous, 16-byte aligned tensors")
    new_k, new_v = (t if _hip.layout_ok(t) else t.contiguous() for t in (new_k, new_v))
    out, lse = _append_decode(q, k_cache, v_cache, new_k, new_v, seqlens, 0, max(host_lengths),
                              float(scale), with_lse=with_lse, host_lengths=host_lengths)
    return (out, lse) if with_lse else out


def attention_decode_ragged(q, k_cache, v_cache, seqlens: torch.Tensor, *, max_seqlen: int,
                            scale: float, with_lse: bool = False,
                            host_lengths: Optional[Sequence[int]] = None):
    """Non-causal decode where batch entry b sees cache positions
    [0, seqlens[b]). ``seqlens`` is a device int32 [B] tensor and
    ``max_seqlen`` >= max(seqlens) bounds the planned splits. ``host_lengths``
    (the same lengths on the host, with max == max_seqlen) lets the planner
    size the splits from the total visible work. Returns O, or (O, LSE) with
    ``with_lse``."""
    require_hip_tensors("ragged decode", q, k_cache, v_cache)
    if seqlens.dtype != torch.int32 or seqlens.device != q.device or seqlens.shape != (q.shape[0],):
        raise ValueError("seqlens must be a device int32 tensor of shape [B]")
    if not seqlens.is_contiguous():  # the kernel reads seqlens[b] as a dense array
        seqlens = seqlens.contiguous()
    if q.ndim != 4 or k_cache.ndim != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("expected [B,H,S,D] query and cache tensors")
    if not (0 < max_seqlen <= k_cache.shape[2]):
        raise ValueError("max_seqlen must be in [1, capacity]")
    if q.shape[0] != k_cache.shape[0] or q.shape[1] % k_cache.shape[1] or q.shape[3] != k_cache.shape[3]:
        raise ValueError("query and cache shapes are incompatible")
    d = q.shape[3]
    if d % 8 or not gfx950_head_dim_ok(d):
        raise ValueError("ragged decode needs head_dim a multiple of 8 in [8, 128]")
    k_view = k_cache[:, :, :max_seqlen]
    v_view = v_cache[:, :, :max_seqlen]
    if not all(_hip.layout_ok(t) for t in (q, k_view, v_view)):
        raise ValueError("ragged decode needs inner-contiguous, 16-byte aligned tensors")
    if host_lengths is not None and len(host_lengths) != q.shape[0]:
        raise ValueError("host_lengths must have one entry per batch element")
    out, lse = _decode(q, k_view, v_view, seqlens, float(scale), with_lse=with_lse,
                       host_lengths=host_lengths)
    return (out, lse) if with_lse else out


def lse_merge(part_o: torch.Tensor, part_lse: torch.Tensor, *, dtype: torch.dtype = torch.float16):
    """Merge split-KV partials with their LSE weights (reference
    triton_forward.py:269-349): part_o fp32 [splits, B, H, Sq, D] and part_lse
    fp32 [splits, B, H, Sq] (natural log; -inf marks an empty split) give
    O [B, H, Sq, D] in ``dtype`` and LSE [B, H, Sq] in fp32. One launch of
    kf_lse_merge. The partials may come from anywhere: another GPU's share of
    a sequence-sharded decode, or the reference's own split layout."""
    if not (isinstance(part_o, torch.Tensor) and isinstance(part_lse, torch.Tensor)):
        raise TypeError("part_o and part_lse must be tensors")
    if part_o.ndim != 5 or part_lse.shape != part_o.shape[:4]:
        raise ValueError("part_o must be [splits, B, H, Sq, D] and part_lse [splits, B, H, Sq]")
    if part_o.dtype != torch.float32 or part_lse.dtype != torch.float32:
        raise TypeError("split partials must be float32")
    if not part_o.is_cuda or part_lse.device != part_o.device:
        raise ValueError("split partials must be GPU tensors on one device")
    if dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("the merged output dtype must be float16 or bfloat16")
    d = part_o.shape[-1]
    if d % 4 or not 4 <= d <= 128:
        raise ValueError("head_dim must be a multiple of 4 in [4, 128]")
    if not _hip.is_gfx950(part_o.device):
        raise RuntimeError("lse_merge requires an AMD gfx950 (MI355X) device")
    part_o = part_o.contiguous()
    part_lse = part_lse.contiguous()
    _, b, h, sq, _ = part_o.shape
    out = torch.empty((b, h, sq, d), device=part_o.device, dtype=dtype)
    lse = torch.empty((b, h, sq), device=part_o.device, dtype=torch.float32)
    _hip.lse_merge(part_o, part_lse, out, lse)
    return out, lse
