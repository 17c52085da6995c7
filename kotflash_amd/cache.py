"""Caller-managed K/V caches for incremental decoding.

Drop-in for the reference's ``kotflash.cache`` (kotflash/cache.py:1-290):
``append_kv_cache``, ``decode_step`` and ``PreallocatedKVCache`` keep their
signatures, checks, messages and the validate-before-write rule (a rejected
append leaves ``length`` and the storage untouched). Append backends:
``"torch"`` (two tensor copies), ``"hip"`` (one gfx950 kernel launch for K and
V; ``"cuda"`` is accepted as an alias) and ``"auto"`` (the HIP kernel for
fp16/bf16 caches on gfx950, torch copies otherwise).

``RaggedKVCache`` extends the fixed-capacity cache to per-sequence lengths:
every sequence appends at its own position in one launch and decode masks
each sequence to its own prefix. These helpers do not implement paging,
eviction, batching or model projections.
"""
from __future__ import annotations

import os
from typing import List, Sequence, Tuple, Union

import torch

from . import _hip
from .attention import attention

APPEND_BACKENDS = ("auto", "torch", "hip", "cuda")


def _validate_kv_tensors(k_cache, v_cache, new_k, new_v) -> None:
    """Reference checks for cache + new K/V (kotflash/cache.py:16-39)."""
    tensors = (k_cache, v_cache, new_k, new_v)
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        raise TypeError("K/V cache and new K/V values must be torch.Tensor instances")
    if any(t.ndim != 4 for t in tensors):
        raise ValueError("All K/V tensors must use [B, Hkv, S, D] layout")
    if k_cache.shape != v_cache.shape:
        raise ValueError("K and V cache shapes must match")
    if k_cache.shape[0] <= 0 or k_cache.shape[1] <= 0 or k_cache.shape[3] <= 0:
        raise ValueError("K/V cache batch, head count and head dimension must be non-zero")
    if new_k.shape != new_v.shape:
        raise ValueError("New K and V shapes must match")
    if (k_cache.shape[0] != new_k.shape[0] or k_cache.shape[1] != new_k.shape[1]
            or k_cache.shape[3] != new_k.shape[3]):
        raise ValueError("New K/V batch, head count and head dimension must match the cache")
    if any(t.device != k_cache.device for t in tensors):
        raise ValueError("All K/V tensors must be on the same device")
    if any(t.dtype != k_cache.dtype for t in tensors):
        raise ValueError("All K/V tensors must have the same dtype")
    if new_k.shape[2] == 0:
        raise ValueError("Appended K/V sequence length must be non-zero")


def append_kv_cache(k_cache, v_cache, new_k, new_v) -> Tuple[torch.Tensor, torch.Tensor]:
    """Concatenate [B, Hkv, Snew, D] entries without mutating the old cache
    (reference kotflash/cache.py:42-54). Copies the whole cache; use
    ``PreallocatedKVCache`` for fixed-capacity storage."""
    _validate_kv_tensors(k_cache, v_cache, new_k, new_v)
    return torch.cat((k_cache, new_k), dim=2), torch.cat((v_cache, new_v), dim=2)


def decode_step(q_new, k_cache, v_cache, k_new, v_new, *, backend: str = "auto"):
    """Append one K/V token and attend with one newest query token
    (reference kotflash/cache.py:57-88). The updated cache holds only keys
    visible to the query, so attention is non-causal."""
    _validate_kv_tensors(k_cache, v_cache, k_new, v_new)
    if k_new.shape[2] != 1:
        raise ValueError("decode_step accepts exactly one new K/V token")
    if not isinstance(q_new, torch.Tensor) or q_new.ndim != 4:
        raise ValueError("q_new must use [B, Hq, 1, D] layout")
    if q_new.shape[2] != 1:
        raise ValueError("decode_step accepts exactly one new query token")
    if q_new.shape[0] != k_cache.shape[0] or q_new.shape[-1] != k_cache.shape[-1]:
        raise ValueError("Query batch and head dimension must match the KV cache")
    if q_new.shape[1] <= 0 or q_new.shape[1] % k_cache.shape[1] != 0:
        raise ValueError("Query heads must be non-zero and divisible by the cache KV-head count")
    if q_new.device != k_cache.device or q_new.dtype != k_cache.dtype:
        raise ValueError("Query device and dtype must match the KV cache")
    updated_k = torch.cat((k_cache, k_new), dim=2)
    updated_v = torch.cat((v_cache, v_new), dim=2)
    output = attention(q_new, updated_k, updated_v, causal=False, backend=backend)
    return output, updated_k, updated_v


def _auto_fuses(q: torch.Tensor, cache: torch.Tensor, visible: int, attention_backend: str,
                has_grad: bool) -> bool:
    """Whether ``append_backend="auto"`` takes the fused append + decode: the
    native append is enabled (``_use_hip_append``), there is no autograd, the
    head_dim is a multiple of 8, and the attention backend is the HIP one --
    forced, or ``auto`` routing this decode shape (``visible`` keys after the
    append) to it."""
    if has_grad or attention_backend not in ("auto", "hip", "triton") or q.shape[-1] % 8:
        return False
    if not _use_hip_append("auto", cache):
        return False
    if attention_backend != "auto":
        return True
    from ._planning import gfx950_profile_for_shapes

    k_shape = (cache.shape[0], cache.shape[1], visible, cache.shape[3])
    dtype_name = str(q.dtype).replace("torch.", "")
    return gfx950_profile_for_shapes(tuple(q.shape), k_shape, causal=False,
                                     dtype_name=dtype_name, needs_grad=False) == "hip"


def _use_hip_append(backend: str, cache: torch.Tensor) -> bool:
    if backend in ("hip", "cuda"):
        return True
    if backend != "auto":
        return False
    if os.environ.get("KOTFLASH_ENABLE_CUDA_APPEND") == "0":
        return False
    return (cache.is_cuda and cache.dtype in (torch.float16, torch.bfloat16)
            and _hip.is_gfx950(cache.device) and _hip.library_available())


class PreallocatedKVCache:
    """Fixed-capacity K/V storage with append-only writes (reference
    kotflash/cache.py:91-290).

    ``view()`` returns storage-backed prefix views (not contiguous once the
    cache is partly filled); the HIP decode reads them in place.
    ``contiguous_view()`` copies the populated prefix. Not thread-safe.
    """

    def __init__(self, batch: int, kv_heads: int, max_len: int, head_dim: int, *,
                 device: Union[torch.device, str], dtype: torch.dtype) -> None:
        dims = {"batch": batch, "kv_heads": kv_heads, "max_len": max_len, "head_dim": head_dim}
        for name, value in dims.items():
            if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        self.k = torch.empty((batch, kv_heads, max_len, head_dim), device=device, dtype=dtype)
        self.v = torch.empty_like(self.k)
        self.max_len = max_len
        self.length = 0

    def _check_new(self, new_k, new_v) -> None:
        if not isinstance(new_k, torch.Tensor) or not isinstance(new_v, torch.Tensor):
            raise TypeError("new_k and new_v must be torch.Tensor instances")
        if new_k.ndim != 4 or new_v.ndim != 4:
            raise ValueError("new K/V must use [B, Hkv, S, D] layout")
        if new_k.shape != new_v.shape:
            raise ValueError("new K and V shapes must match")
        if (new_k.shape[0] != self.k.shape[0] or new_k.shape[1] != self.k.shape[1]
                or new_k.shape[3] != self.k.shape[3]):
            raise ValueError("new K/V batch, heads and head_dim must match the cache")
        if new_k.shape[2] <= 0:
            raise ValueError("cannot append an empty K/V sequence")
        if new_k.device != self.k.device or new_v.device != self.v.device:
            raise ValueError("new K/V must be on the cache device")
        if new_k.dtype != self.k.dtype or new_v.dtype != self.v.dtype:
            raise ValueError("new K/V dtype must match the cache dtype")

    def append(self, new_k: torch.Tensor, new_v: torch.Tensor, *, backend: str = "auto") -> None:
        """Append positions after validation (reference cache.py:124-178)."""
        self._check_new(new_k, new_v)
        if backend not in APPEND_BACKENDS:
            raise ValueError("append backend must be one of: auto, torch, hip or cuda")
        end = self.length + new_k.shape[2]
        if end > self.max_len:
            raise ValueError(
                f"KV cache full: {self.length} + {new_k.shape[2]} tokens "
                f"exceeds max_len={self.max_len}"
            )
        # Every check is done; only now is storage written.
        if _use_hip_append(backend, self.k):
            from ._hip_append import append_kv_hip

            append_kv_hip(self.k, self.v, new_k, new_v, self.length)
        else:
            self.k[:, :, self.length:end].copy_(new_k)
            self.v[:, :, self.length:end].copy_(new_v)
        self.length = end

    def view(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Storage-backed views of the populated prefix."""
        if self.length == 0:
            raise ValueError("KV cache is empty")
        return self.k[:, :, : self.length, :], self.v[:, :, : self.length, :]

    def contiguous_view(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Contiguous copies of the populated prefix."""
        k, v = self.view()
        return k.contiguous(), v.contiguous()

    def _check_query(self, q_new) -> None:
        if not isinstance(q_new, torch.Tensor) or q_new.ndim != 4 or q_new.shape[2] != 1:
            raise ValueError("q_new must use [B, Hq, 1, D] layout")
        if q_new.shape[0] != self.k.shape[0] or q_new.shape[-1] != self.k.shape[-1]:
            raise ValueError("Query batch and head dimension must match the cache")
        if q_new.shape[1] <= 0 or q_new.shape[1] % self.k.shape[1] != 0:
            raise ValueError("Query heads must be non-zero and divisible by the cache KV-head count")
        if q_new.device != self.k.device or q_new.dtype != self.k.dtype:
            raise ValueError("Query device and dtype must match the cache")

    def append_and_attend(self, q_new, new_k, new_v, *, append_backend: str = "auto",
                          attention_backend: str = "auto") -> torch.Tensor:
        """Append one token and attend over the cache without copying the
        prefix (reference cache.py:191-277).

        ``append_backend="fused"`` runs the inference-only append + decode
        launcher (the split-KV kernel also stores the token, then the merge);
        it needs an explicit or automatic HIP attention backend and no
        autograd. ``"auto"`` takes it whenever it applies (``_auto_fuses``),
        else appends with the HIP kernel or torch copies and attends.
        """
        if attention_backend not in ("auto", "hip", "triton", "sdpa"):
            raise ValueError("attention backend must be one of: auto, hip, triton or sdpa")
        if append_backend not in ("auto", "torch", "hip", "cuda", "fused"):
            raise ValueError("append backend must be one of: auto, torch, hip, cuda or fused")
        self._check_query(q_new)
        _validate_kv_tensors(self.k, self.v, new_k, new_v)
        if new_k.shape[2] != 1:
            raise ValueError("append_and_attend accepts exactly one new K/V token")
        end = self.length + 1
        if end > self.max_len:
            raise ValueError(
                f"KV cache full: {self.length} + 1 tokens exceeds max_len={self.max_len}"
            )
        has_grad = torch.is_grad_enabled() and any(
            t.requires_grad for t in (q_new, new_k, new_v)
        )
        if append_backend == "fused" or (append_backend == "auto" and _auto_fuses(
                q_new, self.k, end, attention_backend, has_grad)):
            if attention_backend == "sdpa":
                raise ValueError("append_backend='fused' requires attention_backend='auto' or 'hip'")
            if has_grad:
                raise RuntimeError("append_backend='fused' is inference-only; disable gradients")
            from .kernels.hip_decode import attention_forward_strided_append

            output = attention_forward_strided_append(
                q_new, self.k, self.v, new_k, new_v,
                past_length=self.length, scale=1.0 / (self.k.shape[-1] ** 0.5),
            )
            self.length = end
            return output
        self.append(new_k, new_v, backend=append_backend)
        return self.attend(q_new, backend=attention_backend)

    def attend(self, q_new: torch.Tensor, *, backend: str = "auto") -> torch.Tensor:
        """Attend one newest query token to the populated cache."""
        self._check_query(q_new)
        k, v = self.view()
        return attention(q_new, k, v, causal=False, backend=backend)


class RaggedKVCache(PreallocatedKVCache):
    """Fixed-capacity cache whose batch entries have their own lengths.

    ``lengths[b]`` is the number of populated positions of sequence b (kept on
    the host and mirrored in the device tensors ``seqlens`` (int32) and
    ``starts`` (int64) that the kernels read). ``append`` writes
    new[b, :, t] to position lengths[b] + t of every sequence in one launch;
    ``attend`` runs non-causal decode in which query rows of sequence b see
    positions [0, lengths[b]). An extension of the reference, whose cache has
    a single scalar length (kotflash/cache.py:122).
    """

    def __init__(self, batch: int, kv_heads: int, max_len: int, head_dim: int, *,
                 device: Union[torch.device, str], dtype: torch.dtype) -> None:
        super().__init__(batch, kv_heads, max_len, head_dim, device=device, dtype=dtype)
        self.lengths: List[int] = [0] * batch
        self.seqlens = torch.zeros(batch, device=self.k.device, dtype=torch.int32)
        self.starts = torch.zeros(batch, device=self.k.device, dtype=torch.int64)

    def set_lengths(self, lengths: Sequence[int]) -> None:
        """Declare per-sequence lengths for data the caller wrote directly
        into ``k``/``v`` (for example a prefill)."""
        lengths = [int(x) for x in lengths]
        if len(lengths) != self.k.shape[0]:
            raise ValueError("lengths must have one entry per batch element")
        if any(x < 0 or x > self.max_len for x in lengths):
            raise ValueError(f"lengths must be in [0, max_len={self.max_len}]")
        self._set(lengths)

    def _set(self, lengths: List[int]) -> None:
        self.lengths = lengths
        self.length = max(lengths) if lengths else 0
        host = torch.tensor(lengths, dtype=torch.int64)
        self.starts.copy_(host, non_blocking=False)
        self.seqlens.copy_(host.to(torch.int32), non_blocking=False)

    def append(self, new_k: torch.Tensor, new_v: torch.Tensor, *, backend: str = "auto") -> None:
        self._check_new(new_k, new_v)
        if backend not in APPEND_BACKENDS:
            raise ValueError("append backend must be one of: auto, torch, hip or cuda")
        n = new_k.shape[2]
        full = [b for b, x in enumerate(self.lengths) if x + n > self.max_len]
        if full:
            b = full[0]
            raise ValueError(
                f"KV cache full: sequence {b} has {self.lengths[b]} + {n} tokens "
                f"exceeding max_len={self.max_len}"
            )
        if _use_hip_append(backend, self.k):
            from ._hip_append import append_kv_hip

            append_kv_hip(self.k, self.v, new_k, new_v, self.starts, host_starts=self.lengths)
        else:
            for b, start in enumerate(self.lengths):
                self.k[b, :, start:start + n].copy_(new_k[b])
                self.v[b, :, start:start + n].copy_(new_v[b])
        self._set([x + n for x in self.lengths])

    def append_and_attend(self, q_new, new_k, new_v, *, append_backend: str = "auto",
                          attention_backend: str = "auto") -> torch.Tensor:
        """Append n tokens to every sequence, then attend, non-causally, with
        q_new [B, Hq, Sq, D] over each sequence's first lengths[b] + n
        positions.

        ``append_backend="fused"`` stores the new tokens from inside the
        split-KV decode (one decode launch and the merge, no append launch;
        inference only). ``"auto"`` takes it when it applies (``_auto_fuses``);
        otherwise it appends (``append``) and attends (``attend``) as two
        steps.
        """
        if attention_backend not in ("auto", "hip", "triton", "sdpa"):
            raise ValueError("attention backend must be one of: auto, hip, triton or sdpa")
        if append_backend not in ("auto", "torch", "hip", "cuda", "fused"):
            raise ValueError("append backend must be one of: auto, torch, hip, cuda or fused")
        self._check_new(new_k, new_v)
        if not isinstance(q_new, torch.Tensor) or q_new.ndim != 4:
            raise ValueError("q must use [B, Hq, Sq, D] layout")
        if q_new.shape[0] != self.k.shape[0] or q_new.shape[-1] != self.k.shape[-1]:
            raise ValueError("Query batch and head dimension must match the cache")
        if q_new.shape[1] <= 0 or q_new.shape[1] % self.k.shape[1] != 0:
            raise ValueError("Query heads must be non-zero and divisible by the cache KV-head count")
        if q_new.device != self.k.device or q_new.dtype != self.k.dtype:
            raise ValueError("Query device and dtype must match the cache")
        n = new_k.shape[2]
        full = [b for b, x in enumerate(self.lengths) if x + n > self.max_len]
        if full:
            b = full[0]
            raise ValueError(
                f"KV cache full: sequence {b} has {self.lengths[b]} + {n} tokens "
                f"exceeding max_len={self.max_len}"
            )
        has_grad = torch.is_grad_enabled() and any(
            t.requires_grad for t in (q_new, new_k, new_v)
        )
        fused = append_backend == "fused" or (append_backend == "auto" and _auto_fuses(
            q_new, self.k, max(self.lengths) + n, attention_backend, has_grad))
        if fused:
            if attention_backend == "sdpa":
                raise ValueError("append_backend='fused' requires attention_backend='auto' or 'hip'")
            if has_grad:
                raise RuntimeError("append_backend='fused' is inference-only; disable gradients")
            from .kernels.hip_decode import attention_append_decode_ragged

            out = attention_append_decode_ragged(
                q_new, self.k, self.v, new_k, new_v, self.seqlens, host_lengths=self.lengths,
                scale=1.0 / (q_new.shape[-1] ** 0.5),
            )
            self._set([x + n for x in self.lengths])
            return out
        self.append(new_k, new_v, backend=append_backend)
        return self.attend(q_new, backend=attention_backend)

    def view(self, b: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
        """Storage-backed [1, Hkv, lengths[b], D] views of sequence b."""
        if self.lengths[b] == 0:
            raise ValueError("KV cache is empty")
        n = self.lengths[b]
        return self.k[b:b + 1, :, :n, :], self.v[b:b + 1, :, :n, :]

    def attend(self, q: torch.Tensor, *, backend: str = "auto") -> torch.Tensor:
        """Non-causal decode of q [B, Hq, Sq, D]; rows of sequence b see its
        first lengths[b] positions. HIP: one split-KV decode launch for all
        sequences; SDPA: one call per sequence."""
        if not isinstance(q, torch.Tensor) or q.ndim != 4:
            raise ValueError("q must use [B, Hq, Sq, D] layout")
        if q.shape[0] != self.k.shape[0] or q.shape[-1] != self.k.shape[-1]:
            raise ValueError("Query batch and head dimension must match the cache")
        if q.shape[1] <= 0 or q.shape[1] % self.k.shape[1] != 0:
            raise ValueError("Query heads must be non-zero and divisible by the cache KV-head count")
        if q.device != self.k.device or q.dtype != self.k.dtype:
            raise ValueError("Query device and dtype must match the cache")
        if min(self.lengths) == 0:
            raise ValueError("KV cache is empty")
        if backend not in ("auto", "hip", "triton", "sdpa"):
            raise ValueError("backend must be one of: auto, hip, triton, sdpa")
        use_hip = backend in ("hip", "triton") or (
            backend == "auto" and q.is_cuda and _hip.is_gfx950(q.device)
            and q.dtype in (torch.float16, torch.bfloat16) and q.shape[-1] % 8 == 0
        )
        if use_hip:
            from .kernels.hip_decode import attention_decode_ragged

            return attention_decode_ragged(
                q, self.k, self.v, self.seqlens, max_seqlen=max(self.lengths),
                scale=1.0 / (q.shape[-1] ** 0.5), host_lengths=self.lengths,
            )
        outs = []
        for b in range(q.shape[0]):
            kb, vb = self.view(b)
            outs.append(attention(q[b:b + 1], kb, vb, causal=False, backend="sdpa"))
        return torch.cat(outs, dim=0)
