"""Forward parity on the GPU: HIP kernel (through the C ABI) vs the oracle,
the golden fixtures and fp32 references, at test shapes and at the BASELINE
configurations."""
import math

import numpy as np
import pytest
import torch

from kotflash_amd import attention
from kotflash_amd.kernels.hip_forward import attention_forward
from oracle import attention_oracle as orc
from tests.conftest import GOLDEN_ATTN_CASES
from tests.gpu_helpers import FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


@pytest.mark.parametrize("name", GOLDEN_ATTN_CASES)
def test_forward_matches_golden(golden, name):
    b, hq, hkv, sq, sk, d, causal = (int(x) for x in golden[f"{name}/meta"])
    q, k, v = (torch.from_numpy(golden[f"{name}/{x}"]).cuda() for x in ("q", "k", "v"))
    out, lse = attention_forward(q, k, v, causal=bool(causal), scale=1 / math.sqrt(d))
    assert_close(out, torch.from_numpy(golden[f"{name}/o"]), **FWD_TOL[F16], what=f"{name} O")
    assert_close(lse, torch.from_numpy(golden[f"{name}/lse"]), **FWD_TOL[F16], what=f"{name} LSE")


def test_config1_matches_oracle():
    """B=2, Hq=8, Hkv=2, S=512, D=64, causal, fp16 on GPU,
    against the float64 oracle on the same fp16-rounded inputs (P rounded to
    fp16 like the kernels)."""
    q = seeded((2, 8, 512, 64), 1, dtype=F16)
    k = seeded((2, 2, 512, 64), 2, dtype=F16)
    v = seeded((2, 2, 512, 64), 3, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=True, scale=0.125)
    eo, el = orc.forward_blockwise(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(),
                                   causal=True, scale=0.125, p_dtype=np.float16)
    assert_close(out, torch.from_numpy(eo), **FWD_TOL[F16], what="cfg1 O")
    assert_close(lse, torch.from_numpy(el), **FWD_TOL[F16], what="cfg1 LSE")


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("head_dim", [32, 64, 72, 96, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_head_dims_gqa(dtype, head_dim, causal):
    """The reference's forward case (tests/test_triton.py:19-32): Sq=129,
    Sk=161, Hq=8, Hkv=2."""
    q = seeded((1, 8, 129, head_dim), 11, dtype=dtype)
    k = seeded((1, 2, 161, head_dim), 12, dtype=dtype)
    v = seeded((1, 2, 161, head_dim), 13, dtype=dtype)
    out, lse = attention_forward(q, k, v, causal=causal, scale=1 / math.sqrt(head_dim))
    eo, el = reference_fp32(q, k, v, causal=causal)
    assert_close(out, eo, **FWD_TOL[dtype], what="O")
    assert_close(lse, el, **FWD_TOL[dtype], what="LSE")


@pytest.mark.parametrize("shape", [
    # (B, Hq, Hkv, Sq, Sk, D, causal)
    (1, 1, 1, 1, 1, 64, True),
    (1, 2, 1, 1, 700, 64, True),       # one query row, causal: sees key 0 only
    (2, 4, 4, 300, 1, 32, False),      # one key
    (1, 4, 1, 500, 130, 64, True),     # Sq > Sk causal: late rows see every key
    (1, 2, 2, 70, 900, 128, True),     # Sq < Sk causal: upper-left mask
    (3, 6, 3, 257, 255, 96, False),    # ragged tile edges
    (1, 2, 1, 65, 65, 8, True),        # smallest head_dim
    (1, 2, 1, 33, 47, 20, False),      # head_dim padded 20 -> 24
    (1, 3, 1, 40, 40, 100, True),      # head_dim padded 100 -> 104 (DT 128)
    (1, 32, 1, 128, 256, 64, False),   # MQA, 32 query heads
])
def test_forward_edge_shapes(shape):
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 21, dtype=F16)
    k = seeded((b, hkv, sk, d), 22, dtype=F16)
    v = seeded((b, hkv, sk, d), 23, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=causal, scale=1 / math.sqrt(d))
    eo, el = reference_fp32(q, k, v, causal=causal)
    assert out.shape == q.shape and lse.shape == q.shape[:3]
    assert_close(out, eo, **FWD_TOL[F16], what=f"O {shape}")
    assert_close(lse, el, **FWD_TOL[F16], what=f"LSE {shape}")


@pytest.mark.parametrize("shape", [
    # (B, Hq, Hkv, Sq, Sk, D, causal, dtype). The launcher takes the split
    # form (four waves share a 32-row block's key range) while Sk > 128 and
    # B * Hq * ceil(Sq / 128) <= 128 (causal) or 64 (non-causal), the 128-row
    # tiled form otherwise; ragged edges on both sides of that line.
    (1, 128, 32, 100, 300, 64, True, F16),     # split, at the causal limit
    (1, 129, 43, 100, 300, 64, True, F16),     # tiled, one tile past it
    (2, 20, 4, 300, 257, 128, True, F16),      # split, one-stage rings, Sq > Sk
    (2, 40, 8, 257, 300, 128, True, F16),      # tiled, Sq < Sk
    (2, 40, 8, 257, 200, 96, False, F16),      # tiled, Sq > Sk
    (1, 8, 2, 1000, 1000, 32, True, F16),      # split, 32-wide tile
    (1, 32, 8, 129, 1100, 64, False, F16),     # split, at the limit; waves of 4-5 tiles
    (1, 33, 11, 129, 1100, 64, False, F16),    # tiled, one tile past it
    (1, 8, 2, 700, 700, 128, True, BF16),      # split, bf16
    (1, 6, 3, 90, 1000, 72, False, BF16),      # split, 96-wide tile with 5 k-steps
])
def test_forward_split_and_tiled_forms(shape):
    b, hq, hkv, sq, sk, d, causal, dtype = shape
    q = seeded((b, hq, sq, d), 24, dtype=dtype)
    k = seeded((b, hkv, sk, d), 25, dtype=dtype)
    v = seeded((b, hkv, sk, d), 26, dtype=dtype)
    out, lse = attention_forward(q, k, v, causal=causal, scale=1 / math.sqrt(d))
    eo, el = reference_fp32(q, k, v, causal=causal)
    assert_close(out, eo, **FWD_TOL[dtype], what=f"O {shape}")
    assert_close(lse, el, **FWD_TOL[dtype], what=f"LSE {shape}")


def test_forward_reads_strided_views_in_place():
    """q/k/v as [B, S, H, D] storage viewed as [B, H, S, D] (no copy)."""
    base_q = seeded((2, 200, 8, 64), 31, dtype=F16)
    base_k = seeded((2, 150, 2, 64), 32, dtype=F16)
    base_v = seeded((2, 150, 2, 64), 33, dtype=F16)
    q, k, v = (t.transpose(1, 2) for t in (base_q, base_k, base_v))
    assert not q.is_contiguous()
    out, lse = attention_forward(q, k, v, causal=True, scale=0.125)
    eo, el = reference_fp32(q, k, v, causal=True)
    assert_close(out, eo, **FWD_TOL[F16], what="strided O")
    assert_close(lse, el, **FWD_TOL[F16], what="strided LSE")


def test_custom_scale():
    q = seeded((1, 4, 100, 64), 41, dtype=F16)
    k = seeded((1, 2, 120, 64), 42, dtype=F16)
    v = seeded((1, 2, 120, 64), 43, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=False, scale=0.05)
    eo, el = reference_fp32(q, k, v, causal=False, scale=0.05)
    assert_close(out, eo, **FWD_TOL[F16], what="O")
    assert_close(lse, el, **FWD_TOL[F16], what="LSE")


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_config3_forward(dtype):
    """BASELINE config 3 forward: B=2, Hq=16, Hkv=4, S=4096, D=128, causal,
    q/k/v ~ 0.5 N(0,1)."""
    q = seeded((2, 16, 4096, 128), 301, dtype=dtype, scale=0.5)
    k = seeded((2, 4, 4096, 128), 302, dtype=dtype, scale=0.5)
    v = seeded((2, 4, 4096, 128), 303, dtype=dtype, scale=0.5)
    out, lse = attention_forward(q, k, v, causal=True, scale=1 / math.sqrt(128))
    eo, el = reference_fp32(q, k, v, causal=True)
    assert_close(out, eo, **FWD_TOL[dtype], what="cfg3 O")
    assert_close(lse, el, **FWD_TOL[dtype], what="cfg3 LSE")


@pytest.mark.parametrize("head_dim", [72, 96])
def test_config4_forward(head_dim):
    """BASELINE config 4 forward: B=4, H=12, S=2048, non-causal MHA."""
    q = seeded((4, 12, 2048, head_dim), 401, dtype=F16)
    k = seeded((4, 12, 2048, head_dim), 402, dtype=F16)
    v = seeded((4, 12, 2048, head_dim), 403, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=False, scale=1 / math.sqrt(head_dim))
    eo, el = reference_fp32(q, k, v, causal=False)
    assert_close(out, eo, **FWD_TOL[F16], what="cfg4 O")
    assert_close(lse, el, **FWD_TOL[F16], what="cfg4 LSE")


def test_forward_is_deterministic():
    q = seeded((2, 8, 600, 64), 51, dtype=F16)
    k = seeded((2, 2, 600, 64), 52, dtype=F16)
    v = seeded((2, 2, 600, 64), 53, dtype=F16)
    a = attention_forward(q, k, v, causal=True, scale=0.125)
    b = attention_forward(q, k, v, causal=True, scale=0.125)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_public_attention_routes_to_hip(dtype):
    """Large enough for ``auto`` to take the HIP kernels (>= 1.5e9 FLOP)."""
    q = seeded((2, 8, 1100, 64), 61, dtype=dtype)
    k = seeded((2, 2, 1100, 64), 62, dtype=dtype)
    v = seeded((2, 2, 1100, 64), 63, dtype=dtype)
    for backend in ("auto", "hip", "triton"):
        out = attention(q, k, v, causal=True, backend=backend)
        eo, _ = reference_fp32(q, k, v, causal=True)
        assert_close(out, eo, **FWD_TOL[dtype], what=backend)
    maps = open("/proc/self/maps").read()
    assert "libkotflash_amd.so" in maps


def test_auto_routing_by_problem_size(monkeypatch):
    """``auto`` sends host-bound small training calls to SDPA, and larger
    ones, inference calls of any size and split-KV decode to the HIP
    kernels."""
    import sys

    api = sys.modules["kotflash_amd.attention"]  # the package attribute is the function
    calls = []
    real = api._sdpa

    def counting_sdpa(*args, **kwargs):
        calls.append(args[0].shape)
        return real(*args, **kwargs)

    monkeypatch.setattr(api, "_sdpa", counting_sdpa)
    small = [seeded((2, 8 if i == 0 else 2, 512, 64), 70 + i, dtype=F16) for i in range(3)]
    big = [seeded((2, 8 if i == 0 else 2, 1024, 64), 80 + i, dtype=F16) for i in range(3)]
    dec = [seeded((2, 8 if i == 0 else 2, 1 if i == 0 else 2048, 64), 90 + i, dtype=F16)
           for i in range(3)]
    attention(*small, causal=True)          # inference: HIP at any size
    assert len(calls) == 0
    train = [t.clone().requires_grad_(True) for t in small]
    attention(*train, causal=True)          # small training call: SDPA
    assert len(calls) == 1
    attention(*big, causal=True)
    attention(*[t.clone().requires_grad_(True) for t in big], causal=True)
    attention(*dec, causal=False)
    assert len(calls) == 1
