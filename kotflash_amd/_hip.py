"""ctypes binding of ``libkotflash_amd.so``, the C ABI declared in
``include/kotflash_amd.h``.

This module is the host launcher layer of the reference (the functions that
allocate outputs with torch and launch kernels on the current stream; reference
kotflash/kernels/triton_forward.py:372-456, triton_backward.py:335-421,
triton_decode.py:302-468, kotflash/_cuda_append.py:31-44). Tensors stay torch
tensors; only raw device pointers, sizes, strides and the HIP stream of
PyTorch's current stream cross the boundary. There is no CPU fallback here: if
the library is missing or a call fails, a RuntimeError is raised.
"""
from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libkotflash_amd.so"
ABI_VERSION = 6
KF_F16, KF_BF16 = 0, 1
KF_BWD_DELTA, KF_BWD_DQ, KF_BWD_DKDV, KF_BWD_DKDV_FIXUP = 1, 2, 4, 8
KF_BWD_ALL = KF_BWD_DELTA | KF_BWD_DQ | KF_BWD_DKDV | KF_BWD_DKDV_FIXUP

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_I64P = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "kf_last_error": (ctypes.c_char_p, []),
    "kf_abi_version": (_I, []),
    "kf_attn_fwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                         _I64P, _I64P, _I64P, _I64P, _F, _I, _I, _P]),
    "kf_attn_bwd_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I]),
    "kf_attn_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                         _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                         _F, _I, _I, _P, _SZ, _P]),
    "kf_attn_bwd_stages": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                _I64, _I64, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                                _I64P, _F, _I, _I, _P, _SZ, _P]),
    "kf_decode_num_splits": (_I, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "kf_decode_num_splits_ragged": (_I, [_I64, _I64, _I64, _I64, ctypes.POINTER(ctypes.c_int32),
                                         _I64]),
    "kf_decode_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I]),
    "kf_attn_decode": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                            _I64P, _I64P, _I64P, _I64P, _F, _I, _I, _P, _SZ, _P]),
    "kf_lse_merge": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64P, _I, _P]),
    "kf_attn_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                    _I64P, _I64P, _I64P, _I64P, _F, _I, _I, _P]),
    "kf_kv_append": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                          _I64P, _I64P, _I64P, _I64P, _I, _P]),
    "kf_attn_append_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P, _I64P, _I64P,
                                   _I64P, _F, _I, _I, _P, _SZ, _P]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    """Load the library (after torch, so it binds to torch's HIP runtime)."""
    if not LIB_PATH.is_file():
        raise RuntimeError(
            f"kotflash_amd HIP library not found at {LIB_PATH}; "
            "build it with `python -m kotflash_amd.build`"
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.kf_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"kotflash_amd ABI mismatch: library {version}, bindings {ABI_VERSION}")
    return handle


def library_available() -> bool:
    try:
        lib()
    except (OSError, RuntimeError):
        return False
    return True


@lru_cache(maxsize=16)
def device_arch(index: int) -> str:
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


_GFX950_BY_INDEX: dict = {}


def is_gfx950(device: torch.device) -> bool:
    if device.type != "cuda":
        return False
    index = device.index
    hit = _GFX950_BY_INDEX.get(index)
    if hit is not None:
        return hit
    if not torch.cuda.is_available():
        return False
    dev_index = index if index is not None else torch.cuda.current_device()
    result = device_arch(dev_index) == "gfx950"
    if index is not None:
        _GFX950_BY_INDEX[index] = result  # explicit indices never change meaning
    return result


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return KF_F16
    if dtype == torch.bfloat16:
        return KF_BF16
    raise TypeError(f"HIP kernels support float16 and bfloat16, got {dtype}")


_I64x4 = ctypes.c_int64 * 4
_STRIDE_ARRAYS: dict = {}


def _strides(t: torch.Tensor):
    """The tensor's strides as a ctypes int64[4] (passed where the C ABI
    takes ``const int64_t*``; ctypes hands over the array's address). The
    library only reads them during the call, so one array per distinct
    stride tuple is kept and reused (decode calls repeat the same few)."""
    st = t.stride()
    arr = _STRIDE_ARRAYS.get(st)
    if arr is None:
        if len(_STRIDE_ARRAYS) > 4096:
            _STRIDE_ARRAYS.clear()
        arr = _STRIDE_ARRAYS[st] = _I64x4(*st)
    return arr


_WORKSPACES: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A byte buffer of at least ``nbytes`` for a launch on the current
    stream of ``device``. Launches on one stream run in order, so the stream
    reuses one buffer (grown when needed); another stream gets its own, as
    torch's caching allocator would hand it. During graph capture the buffer
    is a fresh allocation from the graph's pool, so no cached buffer is baked
    into a graph."""
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(nbytes, 256), device=device, dtype=torch.uint8)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, _stream(device))
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is None and len(_WORKSPACES) >= 64:
            # Callers that make a new stream per call would otherwise grow
            # this without bound. Dropping the references is safe: torch's
            # caching allocator only hands a freed block to later work on the
            # stream it was allocated for.
            _WORKSPACES.clear()
        buf = torch.empty(max(nbytes, 256), device=torch.device("cuda", index), dtype=torch.uint8)
        _WORKSPACES[key] = buf
    return buf


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().kf_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """PyTorch's current HIP stream on ``device``, as a raw handle."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


class _DeviceGuard:
    """Makes ``device`` current for a launch; free when it already is (the
    usual case), unlike torch.cuda.device's unconditional exchange."""

    __slots__ = ("index", "prev")

    def __init__(self, device: torch.device):
        self.index = device.index if device.index is not None else -1
        self.prev = -1

    def __enter__(self):
        if self.index >= 0:
            cur = torch.cuda.current_device()
            if cur != self.index:
                self.prev = cur
                torch.cuda.set_device(self.index)
        return self

    def __exit__(self, *exc):
        if self.prev >= 0:
            torch.cuda.set_device(self.prev)
        return False


def layout_ok(t: torch.Tensor) -> bool:
    """Whether the kernels can read ``t`` in place: unit head_dim stride,
    other strides multiples of 8 elements, 16-byte aligned base."""
    s = t.stride()
    if len(s) != 4 or s[3] != 1 or s[0] % 8 or s[1] % 8 or s[2] % 8:
        return False
    return t.data_ptr() % 16 == 0


def fwd(q, k, v, out, lse, *, causal: bool, scale: float) -> None:
    b, hq, sq, d = q.shape
    _, hkv, sk, _ = k.shape
    keep = [_strides(t) for t in (q, k, v, out)]
    with _DeviceGuard(q.device):
        rc = lib().kf_attn_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
            b, hq, hkv, sq, sk, d, *keep,
            float(scale), int(bool(causal)), dtype_code(q.dtype), _stream(q.device),
        )
    _check(rc, "kf_attn_fwd")


@lru_cache(maxsize=256)
def bwd_workspace_bytes(b, hq, hkv, sq, sk, d, causal) -> int:
    return int(lib().kf_attn_bwd_workspace_bytes(b, hq, hkv, sq, sk, d, int(bool(causal))))


def bwd(q, k, v, out, lse, dout, dq, dk, dv, *, causal: bool, scale: float,
        workspace: torch.Tensor, stages: int = KF_BWD_ALL) -> None:
    b, hq, sq, d = q.shape
    _, hkv, sk, _ = k.shape
    keep = [_strides(t) for t in (q, k, v, out, dout, dq, dk, dv)]
    with _DeviceGuard(q.device):
        rc = lib().kf_attn_bwd_stages(
            int(stages), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
            dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
            b, hq, hkv, sq, sk, d, *keep,
            float(scale), int(bool(causal)), dtype_code(q.dtype),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            _stream(q.device),
        )
    _check(rc, "kf_attn_bwd")


@lru_cache(maxsize=256)
def decode_num_splits(b, hq, hkv, sq, sk, d) -> int:
    return int(lib().kf_decode_num_splits(b, hq, hkv, sq, sk, d))


def decode_num_splits_ragged(b, hq, hkv, sq, lengths, d) -> int:
    """Split count for a ragged batch from its host-side visible lengths."""
    lens = (ctypes.c_int32 * len(lengths))(*[int(x) for x in lengths])
    return int(lib().kf_decode_num_splits_ragged(b, hq, hkv, sq, lens, d))


@lru_cache(maxsize=256)
def decode_workspace_bytes(b, hq, hkv, sq, d, num_splits) -> int:
    return int(lib().kf_decode_workspace_bytes(b, hq, hkv, sq, d, num_splits))


def decode(q, k, v, out, lse: Optional[torch.Tensor], seqlens: Optional[torch.Tensor], *,
           scale: float, num_splits: int, workspace: Optional[torch.Tensor]) -> None:
    b, hq, sq, d = q.shape
    _, hkv, sk, _ = k.shape
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.nbytes if workspace is not None else 0
    dev = q.device
    with _DeviceGuard(dev):
        rc = lib().kf_attn_decode(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            lse.data_ptr() if lse is not None else None,
            seqlens.data_ptr() if seqlens is not None else None,
            b, hq, hkv, sq, sk, d, _strides(q), _strides(k), _strides(v), _strides(out),
            float(scale), int(num_splits), dtype_code(q.dtype), ws_ptr, ws_bytes,
            _stream(dev),
        )
    if rc:
        _check(rc, "kf_attn_decode")


def lse_merge(part_o, part_lse, out, lse: Optional[torch.Tensor]) -> None:
    """kf_lse_merge: O (and LSE) from fp32 split partials part_o [S', B, H,
    Sq, D] and part_lse [S', B, H, Sq]."""
    ns, b, h, sq, d = part_o.shape
    keep = _strides(out)
    with _DeviceGuard(out.device):
        rc = lib().kf_lse_merge(
            part_o.data_ptr(), part_lse.data_ptr(), out.data_ptr(),
            lse.data_ptr() if lse is not None else None, ns, b, h, sq, d, keep,
            dtype_code(out.dtype), _stream(out.device),
        )
    _check(rc, "kf_lse_merge")


NOALLOC_SCRATCH_BYTES = 32 << 20  # KF_DECODE_NOALLOC_SCRATCH_BYTES


def decode_noalloc(q, k, v, out, lse: Optional[torch.Tensor], seqlens: Optional[torch.Tensor], *,
                   scale: float, num_splits: int) -> None:
    """kf_attn_decode_noalloc: the split-KV decode with its partials in the
    library's static per-device scratch instead of a workspace (no device
    allocation anywhere in the call; calls overlapping on one GPU race)."""
    b, hq, sq, d = q.shape
    _, hkv, sk, _ = k.shape
    keep = [_strides(t) for t in (q, k, v, out)]
    with _DeviceGuard(q.device):
        rc = lib().kf_attn_decode_noalloc(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            lse.data_ptr() if lse is not None else None,
            seqlens.data_ptr() if seqlens is not None else None,
            b, hq, hkv, sq, sk, d, *keep,
            float(scale), int(num_splits), dtype_code(q.dtype), _stream(q.device),
        )
    _check(rc, "kf_attn_decode_noalloc")


def kv_append(k_cache, v_cache, new_k, new_v, *, start: int = 0,
              start_dev: Optional[torch.Tensor] = None, max_start: Optional[int] = None) -> None:
    """kf_kv_append at the scalar ``start``, or at the per-sequence device
    positions ``start_dev`` (int64 [B]) whose host-side maximum is
    ``max_start``; the library rejects the call before launching unless the
    range ends inside the capacity."""
    b, h, s, d = new_k.shape
    if start_dev is not None:
        if max_start is None:
            raise ValueError("kv_append with start_dev needs max_start, the host-side bound")
        start = max_start
    keep = [_strides(t) for t in (k_cache, v_cache, new_k, new_v)]
    with _DeviceGuard(k_cache.device):
        rc = lib().kf_kv_append(
            k_cache.data_ptr(), v_cache.data_ptr(), new_k.data_ptr(), new_v.data_ptr(),
            start_dev.data_ptr() if start_dev is not None else None, int(start),
            b, h, s, d, k_cache.shape[2], *keep,
            dtype_code(k_cache.dtype), _stream(k_cache.device),
        )
    _check(rc, "kf_kv_append")


def append_decode(q, k_cache, v_cache, new_k, new_v, out, lse: Optional[torch.Tensor],
                  lengths: Optional[torch.Tensor], *, past_length: int, max_length: int,
                  scale: float, num_splits: int, workspace: torch.Tensor) -> None:
    """kf_attn_append_decode: store new_k/new_v at each sequence's position
    and decode over the old keys plus the new ones, in one decode launch."""
    b, hq, sq, d = q.shape
    _, hkv, capacity, _ = k_cache.shape
    keep = [_strides(t) for t in (q, k_cache, v_cache, new_k, new_v, out)]
    with _DeviceGuard(q.device):
        rc = lib().kf_attn_append_decode(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), new_k.data_ptr(),
            new_v.data_ptr(), out.data_ptr(), lse.data_ptr() if lse is not None else None,
            lengths.data_ptr() if lengths is not None else None, int(past_length),
            b, hq, hkv, sq, new_k.shape[2], int(max_length), capacity, d, *keep,
            float(scale), int(num_splits), dtype_code(q.dtype), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), _stream(q.device),
        )
    _check(rc, "kf_attn_append_decode")
