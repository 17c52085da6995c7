"""Pure-Python launch planning and routing tables (no torch imports).

The T4 functions keep the reference's outputs exactly (reference
kotflash/_planning.py:8-76; values pinned by its tests/test_planning.py:17-85).
The gfx950 functions below them are this build's own: the envelope in which the
HIP kernels are used by ``backend="auto"`` on MI355X.
"""
from __future__ import annotations

import math
from typing import NamedTuple, Optional, Sequence

INT32_MAX = 2**31 - 1


def cdiv(a: int, b: int) -> int:
    """Ceiling division for a >= 0, b > 0 (reference _planning.py:11-14)."""
    if a < 0 or b <= 0:
        raise ValueError("cdiv expects a >= 0 and b > 0")
    return -(-a // b)


class SplitKVPlan(NamedTuple):
    block_m: int
    block_n: int
    num_splits: int
    chunk_n: int
    blocks_per_split: int


def split_kv_plan(sq: int, sk: int, d: int, *, causal: bool) -> Optional[SplitKVPlan]:
    """The reference's short-query/long-cache split plan (reference
    _planning.py:25-34): None unless non-causal, Sq <= 16, Sk >= 1024 and
    D <= 64; otherwise at most 16 splits of 64-key blocks."""
    if min(sq, sk, d) <= 0:
        raise ValueError("sq, sk and d must be positive")
    if causal or sq > 16 or sk < 1024 or d > 64:
        return None
    splits = min(16, cdiv(sk, 128))
    chunk = cdiv(sk, splits)
    return SplitKVPlan(16, 64, splits, chunk, cdiv(chunk, 64))


def check_int32_indexing(**numels: int) -> None:
    """Reject element counts above INT32_MAX (reference _planning.py:37-46).

    The HIP kernels index with 64-bit tensor offsets and do not need this
    guard; it is kept for callers of the reference API."""
    for name, n in numels.items():
        if isinstance(n, bool) or not isinstance(n, int) or n < 0:
            raise ValueError(f"{name} must be a non-negative integer element count")
        if n > INT32_MAX:
            raise ValueError(
                f"{name} has {n} elements; Triton kernels use 32-bit offsets "
                f"(limit {INT32_MAX}). Reduce batch/sequence size or use backend='sdpa'."
            )


# Exact shapes the reference measured on a T4 (reference _planning.py:49-54).
_DECODE_PROFILE = {
    ((2, 8, 1, 64), (2, 2, 2048, 64)): "triton",
    ((2, 8, 4, 64), (2, 2, 1024, 64)): "sdpa_expanded",
    ((2, 8, 16, 64), (2, 2, 4096, 64)): "triton",
}
_CAUSAL_LENGTHS = {128, 256, 512, 1024, 2048}


def t4_profile_for_shapes(
    q_shape: Sequence[int], k_shape: Sequence[int], v_shape: Sequence[int], *,
    causal: bool, scale: float, contiguous: bool,
) -> Optional[str]:
    """Backend measured for an exact T4 shape, else None (reference
    _planning.py:57-76)."""
    q_shape, k_shape, v_shape = tuple(q_shape), tuple(k_shape), tuple(v_shape)
    if not contiguous or v_shape != k_shape:
        return None
    if not math.isclose(scale, 0.125, rel_tol=0.0, abs_tol=1e-12):
        return None
    if not causal:
        return _DECODE_PROFILE.get((q_shape, k_shape))
    if len(q_shape) != 4 or len(k_shape) != 4:
        return None
    seq = q_shape[2]
    if q_shape == (2, 8, seq, 64) and k_shape == (2, 2, seq, 64) and seq in _CAUSAL_LENGTHS:
        return "triton" if seq >= 1024 else "sdpa_expanded"
    return None


# ---------------------------------------------------------------------------
# gfx950 (MI355X) routing.

GFX950_MIN_HEAD_DIM = 8
GFX950_MAX_HEAD_DIM = 128
# Split-KV decode envelope: short query against a long cache, non-causal.
GFX950_DECODE_MAX_SQ = 16
GFX950_DECODE_MIN_SK = 1024


def gfx950_head_dim_ok(d: int) -> bool:
    return GFX950_MIN_HEAD_DIM <= d <= GFX950_MAX_HEAD_DIM


def gfx950_decode_eligible(sq: int, sk: int, d: int, *, causal: bool) -> bool:
    """Whether the split-KV decode kernel handles this forward."""
    return (not causal and 0 < sq <= GFX950_DECODE_MAX_SQ and sk >= GFX950_DECODE_MIN_SK
            and gfx950_head_dim_ok(d))


# Below this much forward work (FLOP) an eager training call (forward, then
# backward through autograd) is bound by host time, and PyTorch's SDPA,
# whose launch and autograd paths are C++, finishes first. Measured on MI355X
# through the public API (python -m kotflash_amd.benchmark, B=2 Hq=8 Hkv=2
# D=64 causal, fp16; fwd+bwd us, HIP vs SDPA):
#   S=256: 220 vs 183;  S=512: 216 vs 179;  S=1024: 213 vs 262;
#   S=2048: 261 vs 411 (an earlier run);  B=1 H=8 S=512 D=128 non-causal
#   (1.1e9 FLOP): 215 vs 174.
# Inference calls (no backward to follow) are not subject to it: the HIP
# forward's launch path is the shorter one (config 1, S=512: 18.9 us per call
# against 22.4 us for SDPA, bench.py torch_sdpa_same_gpu), and split-KV decode
# shapes are 22x faster (config 2).
GFX950_HIP_MIN_FWD_FLOPS = 1.5e9


def attention_fwd_flops(q_shape: Sequence[int], k_shape: Sequence[int], *, causal: bool) -> float:
    """4 D B Hq times the visible (query, key) pairs, upper-left causal."""
    b, hq, sq, d = q_shape
    sk = k_shape[2]
    if causal:
        full = max(0, sq - sk)          # rows that see every key
        part = min(sq, sk)              # rows i < sk see i + 1 keys
        pairs = part * (part + 1) // 2 + full * sk
    else:
        pairs = sq * sk
    return 4.0 * d * b * hq * pairs


def gfx950_profile_for_shapes(
    q_shape: Sequence[int], k_shape: Sequence[int], *, causal: bool, dtype_name: str,
    needs_grad: bool = True,
) -> Optional[str]:
    """Backend chosen by ``backend="auto"`` on gfx950, else None (SDPA).

    The HIP kernels cover fp16/bf16 with 8 <= head_dim <= 128 for any
    sequence lengths and GQA grouping. ``auto`` takes them for every
    inference call (``needs_grad=False``), for split-KV decode shapes, and for
    training calls of at least ``GFX950_HIP_MIN_FWD_FLOPS``; smaller training
    calls, and everything outside that envelope, go to SDPA.
    """
    if dtype_name not in ("float16", "bfloat16"):
        return None
    if len(q_shape) != 4 or len(k_shape) != 4:
        return None
    d = q_shape[3]
    if not gfx950_head_dim_ok(d) or k_shape[3] != d:
        return None
    if q_shape[1] % k_shape[1] != 0:
        return None
    if not needs_grad or gfx950_decode_eligible(q_shape[2], k_shape[2], d, causal=causal):
        return "hip"
    if attention_fwd_flops(q_shape, k_shape, causal=causal) < GFX950_HIP_MIN_FWD_FLOPS:
        return None
    return "hip"
