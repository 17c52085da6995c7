"""Pinning the CPU oracle (oracle/attention_oracle.py) before it is trusted.

Every oracle function is checked against something that does not share its
code: the golden fixtures (dense float64 closed form + autograd), closed forms
of special inputs, algebraic invariants, finite differences and slice
assignment. Planted mistakes in oracle variants must fail those checks.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from tests.conftest import GOLDEN_ATTN_CASES


def _case(golden, name):
    meta = golden[f"{name}/meta"]
    b, hq, hkv, sq, sk, d, causal = (int(x) for x in meta)
    q, k, v, do = (golden[f"{name}/{x}"].astype(np.float64) for x in ("q", "k", "v", "do"))
    return q, k, v, do, bool(causal), 1.0 / math.sqrt(d)


@pytest.mark.parametrize("name", GOLDEN_ATTN_CASES)
def test_forward_matches_golden(golden, name):
    q, k, v, _, causal, scale = _case(golden, name)
    out, lse = orc.forward_blockwise(q, k, v, causal=causal, scale=scale, block_m=16, block_n=8)
    np.testing.assert_allclose(out, golden[f"{name}/o"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(lse, golden[f"{name}/lse"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("name", GOLDEN_ATTN_CASES)
def test_backward_matches_golden(golden, name):
    q, k, v, do, causal, scale = _case(golden, name)
    out, lse = orc.forward_blockwise(q, k, v, causal=causal, scale=scale)
    dq, dk, dv = orc.backward_blockwise(q, k, v, out, lse, do, causal=causal, scale=scale,
                                        q_block=7, kv_block=11)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got, golden[f"{name}/{key}"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("bm,bn", [(64, 32), (16, 8), (5, 3), (1, 1)])
def test_forward_tiling_invariant(bm, bn):
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 2, 23, 8))
    k = rng.standard_normal((1, 1, 29, 8))
    v = rng.standard_normal((1, 1, 29, 8))
    ref = orc.forward_blockwise(q, k, v, causal=True, scale=0.3, block_m=64, block_n=64)
    got = orc.forward_blockwise(q, k, v, causal=True, scale=0.3, block_m=bm, block_n=bn)
    np.testing.assert_allclose(got[0], ref[0], atol=1e-12)
    np.testing.assert_allclose(got[1], ref[1], atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_zero_query_closed_form(causal):
    """q = 0: every visible score is 0, so LSE = ln(#visible) and O is the
    mean of the visible V rows (upper-left causal: row i sees i+1 keys)."""
    rng = np.random.default_rng(1)
    sq, sk = 9, 13
    q = np.zeros((1, 2, sq, 4))
    k = rng.standard_normal((1, 1, sk, 4))
    v = rng.standard_normal((1, 1, sk, 4))
    out, lse = orc.forward_blockwise(q, k, v, causal=causal, scale=0.7, block_m=4, block_n=3)
    for i in range(sq):
        n = min(i + 1, sk) if causal else sk
        np.testing.assert_allclose(lse[0, :, i], math.log(n), atol=1e-12)
        np.testing.assert_allclose(out[0, 0, i], v[0, 0, :n].mean(axis=0), atol=1e-12)


def test_causal_first_row_and_constant_v():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 1, 6, 4))
    k = rng.standard_normal((1, 1, 6, 4))
    v = rng.standard_normal((1, 1, 6, 4))
    out, _ = orc.forward_blockwise(q, k, v, causal=True, scale=1.0)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, 0], atol=1e-12)
    const = np.full_like(v, 3.25)
    out2, _ = orc.forward_blockwise(q, k, const, causal=False, scale=1.0)
    np.testing.assert_allclose(out2, 3.25, atol=1e-12)


def test_gqa_head_mapping_matches_per_head_mha():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 6, 5, 4))
    k = rng.standard_normal((1, 2, 7, 4))
    v = rng.standard_normal((1, 2, 7, 4))
    out, _ = orc.forward_blockwise(q, k, v, causal=False, scale=0.5)
    for h in range(6):
        kh = h // 3  # contiguous groups of Hq / Hkv = 3
        o1, _ = orc.forward_blockwise(q[:, h:h + 1], k[:, kh:kh + 1], v[:, kh:kh + 1],
                                      causal=False, scale=0.5)
        np.testing.assert_allclose(out[:, h:h + 1], o1, atol=1e-12)


@pytest.mark.parametrize("splits,chunk", [(1, 300), (3, 100), (7, 43), (16, 19)])
def test_split_merge_equals_unsplit(splits, chunk):
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 4, 3, 8))
    k = rng.standard_normal((2, 2, 300, 8))
    v = rng.standard_normal((2, 2, 300, 8))
    part_o, part_lse = orc.split_kv_partials(q, k, v, scale=0.35, num_splits=splits, chunk_n=chunk)
    out, lse = orc.split_kv_merge(part_o, part_lse)
    ref_o, ref_lse = orc.forward_blockwise(q, k, v, causal=False, scale=0.35)
    np.testing.assert_allclose(out, ref_o, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-12)


def test_empty_split_has_zero_weight_and_all_empty_is_neg_inf():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 2, 1, 4))
    k = rng.standard_normal((2, 1, 40, 4))
    v = rng.standard_normal((2, 1, 40, 4))
    # Batch 0 sees 10 keys: splits 1.. of chunk 10 are empty for it.
    part_o, part_lse = orc.split_kv_partials(q, k, v, scale=1.0, num_splits=4, chunk_n=10,
                                             seqlens=[10, 40])
    assert np.isneginf(part_lse[1:, 0]).all() and (part_o[1:, 0] == 0).all()
    out, lse = orc.split_kv_merge(part_o, part_lse)
    ref0, lse0 = orc.forward_blockwise(q[:1], k[:1, :, :10], v[:1, :, :10], causal=False, scale=1.0)
    np.testing.assert_allclose(out[:1], ref0, atol=1e-12)
    np.testing.assert_allclose(lse[:1], lse0, atol=1e-12)
    o_all, l_all = orc.split_kv_merge(np.zeros((3, 1, 1, 1, 4)), np.full((3, 1, 1, 1), -np.inf))
    assert np.isneginf(l_all).all() and (o_all == 0).all()


def test_split_plan_partitions_without_gaps():
    for sk in list(range(1024, 3000, 7)) + [4096, 8191, 8192, 16384, 20000]:
        splits, chunk, blocks = orc.split_kv_plan(1, sk, 64, causal=False)
        covered = 0
        for s in range(splits):
            start, end = s * chunk, min((s + 1) * chunk, sk)
            assert start == covered and start < end and start + blocks * 64 >= end
            covered = end
        assert covered == sk
    assert orc.split_kv_plan(17, 4096, 64, causal=False) is None
    assert orc.split_kv_plan(1, 1023, 64, causal=False) is None
    assert orc.split_kv_plan(1, 4096, 72, causal=False) is None
    assert orc.split_kv_plan(1, 4096, 64, causal=True) is None


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_finite_differences(causal):
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 2, 4, 3))
    k = rng.standard_normal((1, 1, 5, 3))
    v = rng.standard_normal((1, 1, 5, 3))
    do = rng.standard_normal((1, 2, 4, 3))
    scale = 0.6

    def loss(q_, k_, v_):
        o, _ = orc.forward_blockwise(q_, k_, v_, causal=causal, scale=scale, block_m=2, block_n=2)
        return float((o * do).sum())

    out, lse = orc.forward_blockwise(q, k, v, causal=causal, scale=scale)
    grads = orc.backward_blockwise(q, k, v, out, lse, do, causal=causal, scale=scale,
                                   q_block=3, kv_block=2)
    eps = 1e-6
    for idx, x in enumerate((q, k, v)):
        fd = np.zeros_like(x)
        for pos in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[pos] += eps
            xm[pos] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[idx], args_m[idx] = xp, xm
            fd[pos] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        np.testing.assert_allclose(grads[idx], fd, rtol=1e-6, atol=1e-7)


def test_backward_matches_torch_autograd_gqa():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 4, 9, 8, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 2, 11, 8, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(2, 2, 11, 8, generator=g, dtype=torch.float64, requires_grad=True)
    do = torch.randn(2, 4, 9, 8, generator=g, dtype=torch.float64)
    out = torch.nn.functional.scaled_dot_product_attention(
        q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), is_causal=True)
    ref = torch.autograd.grad(out, (q, k, v), do)
    o, lse = orc.forward_blockwise(q.detach().numpy(), k.detach().numpy(), v.detach().numpy(),
                                   causal=True, scale=1 / math.sqrt(8))
    got = orc.backward_blockwise(q.detach().numpy(), k.detach().numpy(), v.detach().numpy(),
                                 o, lse, do.numpy(), causal=True, scale=1 / math.sqrt(8))
    for a, b in zip(got, ref):
        np.testing.assert_allclose(a, b.numpy(), rtol=1e-9, atol=1e-10)


def test_forward_matches_torch_sdpa_on_cpu():
    g = torch.Generator().manual_seed(8)
    q = torch.randn(2, 8, 19, 16, generator=g)
    k = torch.randn(2, 2, 25, 16, generator=g)
    v = torch.randn(2, 2, 25, 16, generator=g)
    for causal in (False, True):
        ref = orc.sdpa_cpu(q, k, v, causal=causal).numpy()
        got, _ = orc.forward_blockwise(q.numpy(), k.numpy(), v.numpy(), causal=causal,
                                       scale=0.25)
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_append_matches_golden_and_slice_assignment(golden):
    kc = golden["append/k_cache"].copy()
    vc = golden["append/v_cache"].copy()
    orc.kv_append(kc, vc, golden["append/new_k"], golden["append/new_v"],
                  golden["append/starts"])
    assert kc.tobytes() == golden["append/k_expected"].tobytes()
    assert vc.tobytes() == golden["append/v_expected"].tobytes()
    kc2 = golden["append/k_cache"].copy()
    vc2 = golden["append/v_cache"].copy()
    orc.kv_append(kc2, vc2, golden["append/new_k"], golden["append/new_v"], 5)
    ek = golden["append/k_cache"].copy()
    ek[:, :, 5:8] = golden["append/new_k"]
    assert kc2.tobytes() == ek.tobytes()


def test_ragged_golden_against_split_oracle(golden):
    q = golden["ragged/q"].astype(np.float64)
    kc = golden["ragged/k_cache"].astype(np.float64)
    vc = golden["ragged/v_cache"].astype(np.float64)
    lengths = golden["ragged/lengths"]
    part_o, part_lse = orc.split_kv_partials(q, kc, vc, scale=1 / math.sqrt(32), num_splits=5,
                                             chunk_n=32, seqlens=lengths)
    out, lse = orc.split_kv_merge(part_o, part_lse)
    np.testing.assert_allclose(out, golden["ragged/o"], atol=1e-6)
    np.testing.assert_allclose(lse, golden["ragged/lse"], atol=1e-6)


# ---------------------------------------------------------------------------
# Planted mistakes: each variant below is the oracle with one plausible bug; the
# pinning checks above must reject it (otherwise they would pin nothing).

def _forward_strict_causal(q, k, v, scale):
    """Bug: causal mask j < i instead of j <= i."""
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    i = np.arange(q.shape[2])[:, None]
    j = np.arange(k.shape[2])[None, :]
    s = np.where(j < i, s, -np.inf)
    s[..., 0, 0] = 0.0
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ v


def test_planted_mistakes_fail_the_pins(golden):
    name = "gqa_causal_d96"
    q, k, v, do, causal, scale = _case(golden, name)
    ref = golden[f"{name}/o"]
    kk, vv = np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1)
    wrong_mask = _forward_strict_causal(q, kk, vv, scale)
    assert np.abs(wrong_mask - ref).max() > 1e-2
    no_scale, _ = orc.forward_blockwise(q, k, v, causal=causal, scale=1.0)
    assert np.abs(no_scale - ref).max() > 1e-2
    # Untransposed V (V^T used where V is meant) on a square head block.
    sq_case = "cfg1_shape_small"
    q2, k2, v2, _, c2, sc2 = _case(golden, sq_case)
    vt = np.swapaxes(v2, -1, -2).copy()
    bad, _ = orc.forward_blockwise(q2, k2, vt, causal=c2, scale=sc2)
    assert np.abs(bad - golden[f"{sq_case}/o"]).max() > 1e-2
    # Backward without the scale on dK.
    out, lse = orc.forward_blockwise(q, k, v, causal=causal, scale=scale)
    dq, dk, dv = orc.backward_blockwise(q, k, v, out, lse, do, causal=causal, scale=scale)
    assert np.abs(dk / scale - golden[f"{name}/dk"]).max() > 1e-2
