"""Launch planning and routing tables, CPU only.

The T4 routing table and the split plan are part of the reference's public
contract (reference kotflash/_planning.py:8-76). The expected values below are
the ones the reference's own tests pin (its tests/test_planning.py:17-85),
arranged here as one table of routing cases and a brute-force coverage check
of the split plan. The gfx950 functions are this build's own envelope.
"""
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np
import pytest

from kotflash_amd._planning import (
    INT32_MAX, attention_fwd_flops, cdiv, check_int32_indexing, gfx950_decode_eligible,
    gfx950_profile_for_shapes, split_kv_plan, t4_profile_for_shapes,
)


@dataclass(frozen=True)
class RouteCase:
    """One call of t4_profile_for_shapes and the backend it must return."""
    why: str
    q: Tuple[int, ...]
    k: Tuple[int, ...]
    expect: Optional[str]
    causal: bool = True
    scale: float = 0.125          # 1/sqrt(64), the scale of every measured profile
    contiguous: bool = True
    v: Optional[Tuple[int, ...]] = None

    def run(self):
        v = self.k if self.v is None else self.v
        return t4_profile_for_shapes(self.q, self.k, v, causal=self.causal, scale=self.scale,
                                     contiguous=self.contiguous)


def _self_attention(s, d=64, b=2, hq=8, hkv=2):
    return (b, hq, s, d), (b, hkv, s, d)


ROUTES = [
    # The measured causal training profile: B=2, Hq=8, Hkv=2, D=64.
    *(RouteCase(f"causal S={s}", *_self_attention(s), "triton" if s >= 1024 else "sdpa_expanded")
      for s in (128, 256, 512, 1024, 2048)),
    # The measured non-causal decode profile (Sq, Sk).
    RouteCase("decode 1/2048", (2, 8, 1, 64), (2, 2, 2048, 64), "triton", causal=False),
    RouteCase("decode 4/1024", (2, 8, 4, 64), (2, 2, 1024, 64), "sdpa_expanded", causal=False),
    RouteCase("decode 16/4096", (2, 8, 16, 64), (2, 2, 4096, 64), "triton", causal=False),
    # Anything off those exact points is unprofiled: None (SDPA).
    RouteCase("non-causal self-attention", *_self_attention(512), None, causal=False),
    RouteCase("decode, Sk off by one", (2, 8, 4, 64), (2, 2, 1025, 64), None, causal=False),
    RouteCase("decode, Sq not profiled", (2, 8, 2, 64), (2, 2, 2048, 64), None, causal=False),
    RouteCase("decode, Sk not profiled", (2, 8, 1, 64), (2, 2, 4096, 64), None, causal=False),
    RouteCase("non-default scale", *_self_attention(512), None, scale=0.1),
    RouteCase("strided inputs", *_self_attention(512), None, contiguous=False),
    RouteCase("length not profiled", *_self_attention(511), None),
    RouteCase("head_dim 128", *_self_attention(512, d=128), None),
    RouteCase("batch 1", *_self_attention(512, b=1), None),
    RouteCase("16 query heads", *_self_attention(512, hq=16, hkv=4), None),
    RouteCase("length 4096", *_self_attention(4096), None),
    RouteCase("Sk != Sq", (2, 8, 512, 64), (2, 2, 256, 64), None),
    RouteCase("3-D tensors", (8, 512, 64), (2, 512, 64), None),
    RouteCase("V shape differs from K", *_self_attention(512), None, v=(2, 2, 256, 64)),
]


@pytest.mark.parametrize("case", ROUTES, ids=lambda c: c.why)
def test_t4_routing_table(case):
    assert case.run() == case.expect


def _coverage(plan, sk):
    """How many splits claim each key, and whether every split's blocks reach
    its end, recomputed key by key from the plan's fields."""
    hits = np.zeros(sk, dtype=np.int64)
    reach_ok = True
    for s in range(plan.num_splits):
        lo, hi = s * plan.chunk_n, min((s + 1) * plan.chunk_n, sk)
        if lo >= hi:
            return None, False  # an empty split
        hits[lo:hi] += 1
        reach_ok &= lo + plan.blocks_per_split * plan.block_n >= hi
    return hits, reach_ok


@pytest.mark.parametrize("sk", [*range(1024, 3000, 7), 4096, 8191, 8192, 16384, 20000])
def test_split_plan_covers_each_key_exactly_once(sk):
    plan = split_kv_plan(1, sk, 64, causal=False)
    assert plan is not None and (plan.block_m, plan.block_n) == (16, 64)
    assert 1 <= plan.num_splits <= 16
    hits, reach_ok = _coverage(plan, sk)
    assert hits is not None and reach_ok and bool((hits == 1).all())


@pytest.mark.parametrize("sk,splits,chunk", [(2048, 16, 128), (16384, 16, 1024), (1024, 8, 128)])
def test_split_plan_values_at_the_decode_configs(sk, splits, chunk):
    plan = split_kv_plan(1, sk, 64, causal=False)
    assert (plan.num_splits, plan.chunk_n, plan.blocks_per_split) == (splits, chunk, chunk // 64)


@pytest.mark.parametrize("sq,sk,d,causal,why", [
    (1, 1023, 64, False, "cache shorter than 1024"),
    (17, 4096, 64, False, "more than 16 query rows"),
    (1, 4096, 72, False, "head_dim above 64"),
    (1, 4096, 64, True, "causal"),
])
def test_split_plan_envelope(sq, sk, d, causal, why):
    assert split_kv_plan(sq, sk, d, causal=causal) is None, why


@pytest.mark.parametrize("count,ok", [(0, True), (INT32_MAX, True), (INT32_MAX + 1, False)])
def test_int32_guard(count, ok):
    if ok:
        check_int32_indexing(q=count, k=count)
    else:
        with pytest.raises(ValueError, match="32-bit"):
            check_int32_indexing(q=count)


@pytest.mark.parametrize("bad", [True, -1, 2.0])
def test_int32_guard_rejects_non_counts(bad):
    with pytest.raises(ValueError):
        check_int32_indexing(q=bad)


@pytest.mark.parametrize("a,b,want", [(0, 3, 0), (7, 3, 3), (6, 3, 2), (1, 1, 1)])
def test_cdiv(a, b, want):
    assert cdiv(a, b) == want


@pytest.mark.parametrize("a,b", [(1, 0), (-1, 2)])
def test_cdiv_rejects(a, b):
    with pytest.raises(ValueError):
        cdiv(a, b)


def test_gfx950_envelope():
    assert gfx950_profile_for_shapes((2, 16, 4096, 128), (2, 4, 4096, 128), causal=True,
                                     dtype_name="float16") == "hip"
    assert gfx950_profile_for_shapes((2, 16, 4096, 128), (2, 4, 4096, 128), causal=True,
                                     dtype_name="bfloat16") == "hip"
    assert gfx950_profile_for_shapes((2, 16, 64, 128), (2, 4, 64, 128), causal=True,
                                     dtype_name="float32") is None
    assert gfx950_profile_for_shapes((2, 16, 64, 256), (2, 4, 64, 256), causal=False,
                                     dtype_name="float16") is None
    assert gfx950_decode_eligible(1, 16384, 64, causal=False)
    assert gfx950_decode_eligible(16, 1024, 128, causal=False)
    assert not gfx950_decode_eligible(17, 16384, 64, causal=False)
    assert not gfx950_decode_eligible(1, 1023, 64, causal=False)


def test_gfx950_auto_routing_by_size():
    """auto keeps host-bound small problems on SDPA, takes the HIP kernels
    from about 1.5e9 forward FLOP up, and always for split-KV decode."""
    f16 = dict(dtype_name="float16")
    # Config 1: 4 * 64 * 16 * 131328 (the survey's algorithmic work figure).
    assert attention_fwd_flops((2, 8, 512, 64), (2, 2, 512, 64), causal=True) == 537919488
    assert gfx950_profile_for_shapes((2, 8, 512, 64), (2, 2, 512, 64), causal=True, **f16) is None
    assert gfx950_profile_for_shapes((2, 8, 1024, 64), (2, 2, 1024, 64), causal=True, **f16) == "hip"
    assert gfx950_profile_for_shapes((1, 8, 512, 128), (1, 8, 512, 128), causal=False, **f16) is None
    assert gfx950_profile_for_shapes((2, 8, 1, 64), (2, 2, 2048, 64), causal=False, **f16) == "hip"
    # Causal pair count: Sq < Sk (upper-left) and Sq > Sk (late rows see all keys).
    assert attention_fwd_flops((1, 1, 3, 8), (1, 1, 5, 8), causal=True) == 4 * 8 * (1 + 2 + 3)
    assert attention_fwd_flops((1, 1, 5, 8), (1, 1, 3, 8), causal=True) == 4 * 8 * (1 + 2 + 3 + 3 + 3)
    assert not gfx950_decode_eligible(1, 16384, 64, causal=True)


def test_gfx950_auto_routes_inference_calls_to_hip_at_any_size():
    """Without a backward to follow, the HIP forward's launch path is the
    shorter one, so auto takes it below the training threshold too."""
    f16 = dict(dtype_name="float16", needs_grad=False)
    assert gfx950_profile_for_shapes((2, 8, 512, 64), (2, 2, 512, 64), causal=True, **f16) == "hip"
    assert gfx950_profile_for_shapes((1, 1, 8, 8), (1, 1, 8, 8), causal=False, **f16) == "hip"
    # The envelope itself is unchanged: fp32, head_dim 256, bad grouping.
    assert gfx950_profile_for_shapes((2, 8, 512, 64), (2, 2, 512, 64), causal=True,
                                     dtype_name="float32", needs_grad=False) is None
    assert gfx950_profile_for_shapes((1, 2, 8, 256), (1, 2, 8, 256), causal=True, **f16) is None
    assert gfx950_profile_for_shapes((1, 3, 8, 64), (1, 2, 8, 64), causal=True, **f16) is None
