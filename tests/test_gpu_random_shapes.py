"""Forward and backward parity over seeded random shapes: GQA ratios, unequal
and ragged Sq / Sk, head dims from 8 to 128 (padded and tile-tail cases),
causal and not. The shapes fall on both sides of the split-form rule (the
forward and dQ kernels) and give the dK/dV stream-K planner many different
share layouts. fp16 against fp32 autograd at the standard bars, and bf16
against fp32 and PyTorch's own bf16 SDPA."""
import math
import random

import pytest
import torch

from kotflash_amd.kernels.hip_backward import attention_backward
from kotflash_amd.kernels.hip_forward import attention_forward
from tests.gpu_helpers import BWD_TOL, FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _shapes(n=24, seed=2024):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        hkv = rng.choice([1, 2, 3, 4])
        hq = hkv * rng.choice([1, 2, 4, 8])
        b = rng.choice([1, 2, 3])
        sq = rng.randint(1, 2500)
        sk = sq if rng.random() < 0.5 else rng.randint(1, 2500)
        d = rng.choice([8, 16, 40, 64, 72, 80, 96, 104, 128])
        out.append((b, hq, hkv, sq, sk, d, rng.random() < 0.5))
    return out


@pytest.mark.parametrize("shape", _shapes())
def test_random_shape_forward_backward(shape):
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 501, dtype=F16)
    k = seeded((b, hkv, sk, d), 502, dtype=F16)
    v = seeded((b, hkv, sk, d), 503, dtype=F16)
    do = seeded((b, hq, sq, d), 504, dtype=F16)
    scale = 1 / math.sqrt(d)
    out, lse = attention_forward(q, k, v, causal=causal, scale=scale)
    dq, dk, dv = attention_backward(q, k, v, out, lse, do, causal=causal, scale=scale)
    eo, el, (eq, ek, ev) = reference_fp32(q, k, v, causal=causal, with_grad_out=do)
    what = f"{shape}"
    assert_close(out, eo, **FWD_TOL[F16], what=f"{what} O")
    assert_close(lse, el, **FWD_TOL[F16], what=f"{what} LSE")
    assert_close(dq, eq, **BWD_TOL[F16], what=f"{what} dQ")
    assert_close(dk, ek, **BWD_TOL[F16], what=f"{what} dK")
    assert_close(dv, ev, **BWD_TOL[F16], what=f"{what} dV")


BF16 = torch.bfloat16


@pytest.mark.parametrize("shape", _shapes(n=12, seed=4202))
def test_random_shape_bf16(shape):
    """bf16: O and LSE at the bf16 bar; gradients no worse than PyTorch's own
    bf16 SDPA backward on the same inputs (x1.25 + 2e-3), the criterion of
    test_bf16_gradients_no_worse_than_torch: at some shapes the 1e-2 bar is
    at the edge of bf16 itself."""
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 511, dtype=BF16)
    k = seeded((b, hkv, sk, d), 512, dtype=BF16)
    v = seeded((b, hkv, sk, d), 513, dtype=BF16)
    do = seeded((b, hq, sq, d), 514, dtype=BF16)
    scale = 1 / math.sqrt(d)
    out, lse = attention_forward(q, k, v, causal=causal, scale=scale)
    ours = attention_backward(q, k, v, out, lse, do, causal=causal, scale=scale)
    eo, el, exact = reference_fp32(q, k, v, causal=causal, with_grad_out=do)
    assert_close(out, eo, **FWD_TOL[BF16], what=f"{shape} O")
    assert_close(lse, el, **FWD_TOL[BF16], what=f"{shape} LSE")
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    g = hq // hkv
    to = torch.nn.functional.scaled_dot_product_attention(
        qq, kk.repeat_interleave(g, 1).contiguous(), vv.repeat_interleave(g, 1).contiguous(),
        is_causal=causal, scale=scale)
    theirs = torch.autograd.grad(to, (qq, kk, vv), do)
    for a, t, e, n in zip(ours, theirs, exact, "qkv"):
        ea = float((a.float() - e).abs().max())
        et = float((t.float() - e).abs().max())
        assert ea <= 1.25 * et + 2e-3, f"{shape} d{n}: ours {ea:.4f} vs torch {et:.4f}"
