"""Forward and backward parity over seeded random shapes: GQA ratios, unequal
and ragged Sq / Sk, head dims from 8 to 128 (padded and tile-tail cases),
causal and not. The shapes fall on both sides of the split-form rule (the
forward and dQ kernels) and give the dK/dV stream-K planner many different
share layouts. fp16, against fp32 autograd at the standard bars."""
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
