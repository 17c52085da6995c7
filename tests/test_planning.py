"""Planning and routing tables (values from the reference's
tests/test_planning.py:17-85, plus the gfx950 envelope)."""
import pytest

from kotflash_amd._planning import (
    INT32_MAX, attention_fwd_flops, cdiv, check_int32_indexing, gfx950_decode_eligible,
    gfx950_profile_for_shapes, split_kv_plan, t4_profile_for_shapes,
)


def route(q, k, *, causal=True, scale=0.125, contiguous=True, v=None):
    return t4_profile_for_shapes(q, k, k if v is None else v, causal=causal, scale=scale,
                                 contiguous=contiguous)


@pytest.mark.parametrize("seq,expected", [
    (128, "sdpa_expanded"), (256, "sdpa_expanded"), (512, "sdpa_expanded"),
    (1024, "triton"), (2048, "triton"),
])
def test_t4_causal_profile(seq, expected):
    assert route((2, 8, seq, 64), (2, 2, seq, 64)) == expected


@pytest.mark.parametrize("q,k,expected", [
    ((2, 8, 1, 64), (2, 2, 2048, 64), "triton"),
    ((2, 8, 4, 64), (2, 2, 1024, 64), "sdpa_expanded"),
    ((2, 8, 16, 64), (2, 2, 4096, 64), "triton"),
])
def test_t4_decode_profile(q, k, expected):
    assert route(q, k, causal=False) == expected


@pytest.mark.parametrize("q,k,kwargs", [
    ((2, 8, 512, 64), (2, 2, 512, 64), {"causal": False}),
    ((2, 8, 4, 64), (2, 2, 1025, 64), {"causal": False}),
    ((2, 8, 2, 64), (2, 2, 2048, 64), {"causal": False}),
    ((2, 8, 1, 64), (2, 2, 4096, 64), {"causal": False}),
    ((2, 8, 512, 64), (2, 2, 512, 64), {"scale": 0.1}),
    ((2, 8, 512, 64), (2, 2, 512, 64), {"contiguous": False}),
    ((2, 8, 511, 64), (2, 2, 511, 64), {}),
    ((2, 8, 512, 128), (2, 2, 512, 128), {}),
    ((1, 8, 512, 64), (1, 2, 512, 64), {}),
    ((2, 16, 512, 64), (2, 4, 512, 64), {}),
    ((2, 8, 4096, 64), (2, 2, 4096, 64), {}),
    ((2, 8, 512, 64), (2, 2, 256, 64), {}),
    ((8, 512, 64), (2, 512, 64), {}),
])
def test_t4_unprofiled_shapes_fall_back(q, k, kwargs):
    assert route(q, k, **kwargs) is None


def test_t4_mismatched_v_falls_back():
    assert route((2, 8, 512, 64), (2, 2, 512, 64), v=(2, 2, 256, 64)) is None


@pytest.mark.parametrize("sq,sk,d,causal", [
    (1, 1023, 64, False), (17, 4096, 64, False), (1, 4096, 72, False), (1, 4096, 64, True),
])
def test_split_kv_envelope(sq, sk, d, causal):
    assert split_kv_plan(sq, sk, d, causal=causal) is None


def test_split_kv_partitions_without_gaps_or_empty_splits():
    for sk in list(range(1024, 3000, 7)) + [4096, 8191, 8192, 16384, 20000]:
        plan = split_kv_plan(1, sk, 64, causal=False)
        assert plan is not None and 1 <= plan.num_splits <= 16
        covered = 0
        for s in range(plan.num_splits):
            start = s * plan.chunk_n
            end = min(start + plan.chunk_n, sk)
            assert start == covered and start < end
            assert start + plan.blocks_per_split * plan.block_n >= end
            covered = end
        assert covered == sk


def test_int32_guard_and_cdiv():
    check_int32_indexing(q=INT32_MAX)
    with pytest.raises(ValueError, match="32-bit"):
        check_int32_indexing(q=INT32_MAX + 1)
    with pytest.raises(ValueError):
        check_int32_indexing(q=True)
    assert cdiv(0, 3) == 0 and cdiv(7, 3) == 3
    with pytest.raises(ValueError):
        cdiv(1, 0)


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
