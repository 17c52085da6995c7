"""Split-KV decode parity on the GPU (through the C ABI): BASELINE config 2,
the reference's decode cases, padded cache views read in place, ragged
per-sequence lengths (golden fixture) and empty splits."""
import math

import numpy as np
import pytest
import torch

from kotflash_amd import _hip, attention
from kotflash_amd.cache import PreallocatedKVCache
from kotflash_amd.kernels.hip_decode import (
    attention_decode_ragged, attention_forward_strided_decode, strided_decode_supported,
)
from kotflash_amd.kernels.hip_forward import attention_forward
from oracle import attention_oracle as orc
from tests.gpu_helpers import FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


@pytest.mark.parametrize("sk", [2048, 4096, 8192, 16384])
def test_config2_decode(sk):
    """B=2, Hq=8, Hkv=2, Sq=1, D=64, fp16, non-causal."""
    q = seeded((2, 8, 1, 64), 201, dtype=F16)
    k = seeded((2, 2, sk, 64), 202, dtype=F16)
    v = seeded((2, 2, sk, 64), 203, dtype=F16)
    assert strided_decode_supported(q, k, v)
    out, lse = attention_forward(q, k, v, causal=False, scale=0.125)
    eo, el = reference_fp32(q, k, v, causal=False)
    assert_close(out, eo, **FWD_TOL[F16], what="O")
    assert_close(lse, el, **FWD_TOL[F16], what="LSE")
    out2 = attention(q, k, v, causal=False, backend="hip")
    assert torch.equal(out, out2)


def test_config2_small_matches_oracle_split_merge():
    """Split partials + merge of the float64 oracle, with the same split count
    and chunk as the kernel plan."""
    q = seeded((2, 8, 1, 64), 211, dtype=F16)
    k = seeded((2, 2, 2048, 64), 212, dtype=F16)
    v = seeded((2, 2, 2048, 64), 213, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=False, scale=0.125)
    splits = _hip.decode_num_splits(2, 8, 2, 1, 2048, 64)
    chunk = (-(-2048 // splits) + 127) // 128 * 128
    n = lambda t: t.cpu().float().numpy().astype(np.float64)
    po, pl = orc.split_kv_partials(n(q), n(k), n(v), scale=0.125, num_splits=splits, chunk_n=chunk)
    eo, el = orc.split_kv_merge(po, pl)
    assert_close(out, torch.from_numpy(eo), **FWD_TOL[F16], what="O")
    assert_close(lse, torch.from_numpy(el), **FWD_TOL[F16], what="LSE")


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("q_seq,kv_seq,d,hq,hkv", [
    (1, 2048, 64, 8, 2), (4, 1024, 64, 8, 2), (16, 4096, 64, 8, 2),  # test_triton.py:35-53
    (2, 1537, 32, 4, 1), (8, 8193, 32, 4, 1),                       # partial chunks :56-69
    (16, 3000, 128, 32, 1),                                         # MQA: 512 packed rows
    (5, 5000, 96, 12, 4),
])
def test_decode_cases(dtype, q_seq, kv_seq, d, hq, hkv):
    q = seeded((2, hq, q_seq, d), 221, dtype=dtype)
    k = seeded((2, hkv, kv_seq, d), 222, dtype=dtype)
    v = seeded((2, hkv, kv_seq, d), 223, dtype=dtype)
    with torch.no_grad():
        out = attention(q, k, v, causal=False, backend="hip")
    eo, _ = reference_fp32(q, k, v, causal=False)
    assert_close(out, eo, **FWD_TOL[dtype], what="O")


def test_decode_equals_unsplit_forward_at_full_size():
    """Size-independent property: the split-KV result equals the single-pass
    forward kernel's result on the same inputs."""
    q = seeded((2, 8, 1, 64), 231, dtype=F16)
    k = seeded((2, 2, 16384, 64), 232, dtype=F16)
    v = seeded((2, 2, 16384, 64), 233, dtype=F16)
    split_o, split_l = attention_forward(q, k, v, causal=False, scale=0.125)
    o = torch.empty_like(q)
    l_ = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    _hip.fwd(q, k, v, o, l_, causal=False, scale=0.125)
    assert_close(split_o, o, atol=1e-3, rtol=1e-3, what="O")
    assert_close(split_l, l_, atol=1e-4, rtol=1e-5, what="LSE")


def test_preallocated_cache_decode_reads_padded_prefix_in_place():
    """The reference's strided cache case (tests/test_triton.py:212-240): a
    2047-token prefix of a 4096-slot cache, one appended token, NaN in every
    unused slot (any out-of-prefix read would poison the output)."""
    cache = PreallocatedKVCache(2, 2, 4096, 64, device="cuda", dtype=F16)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    pk = seeded((2, 2, 2047, 64), 241, dtype=F16)
    pv = seeded((2, 2, 2047, 64), 242, dtype=F16)
    nk = seeded((2, 2, 1, 64), 243, dtype=F16)
    nv = seeded((2, 2, 1, 64), 244, dtype=F16)
    q = seeded((2, 8, 1, 64), 245, dtype=F16)
    cache.append(pk, pv, backend="hip")
    with torch.inference_mode():
        out = cache.append_and_attend(q, nk, nv, append_backend="hip", attention_backend="hip")
        kv, vv = cache.view()
        assert not kv.is_contiguous()
        assert strided_decode_supported(q, kv, vv)
    eo, _ = reference_fp32(q, kv.contiguous(), vv.contiguous(), causal=False)
    assert torch.isfinite(out).all()
    assert_close(out, eo, **FWD_TOL[F16], what="O")
    out2 = attention_forward_strided_decode(q, kv, vv, scale=0.125)
    assert torch.equal(out, out2)


def test_fused_append_and_attend():
    cache = PreallocatedKVCache(2, 2, 4096, 64, device="cuda", dtype=F16)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    pk = seeded((2, 2, 2047, 64), 251, dtype=F16)
    pv = seeded((2, 2, 2047, 64), 252, dtype=F16)
    nk = seeded((2, 2, 1, 64), 253, dtype=F16)
    nv = seeded((2, 2, 1, 64), 254, dtype=F16)
    q = seeded((2, 8, 1, 64), 255, dtype=F16)
    cache.append(pk, pv, backend="torch")
    with torch.inference_mode():
        out = cache.append_and_attend(q, nk, nv, append_backend="fused", attention_backend="auto")
        torch.cuda.synchronize()
        sk, sv = cache.view()
    assert cache.length == 2048
    assert torch.equal(sk[:, :, -1:], nk) and torch.equal(sv[:, :, -1:], nv)
    eo, _ = reference_fp32(q, torch.cat((pk, nk), 2), torch.cat((pv, nv), 2), causal=False)
    assert_close(out, eo, **FWD_TOL[F16], what="fused O")


def test_ragged_decode_matches_golden(golden):
    q = torch.from_numpy(golden["ragged/q"]).cuda()
    kc = torch.from_numpy(golden["ragged/k_cache"]).cuda()
    vc = torch.from_numpy(golden["ragged/v_cache"]).cuda()
    lengths = torch.from_numpy(golden["ragged/lengths"]).to(torch.int32).cuda()
    out, lse = attention_decode_ragged(q, kc, vc, lengths, max_seqlen=160,
                                       scale=1 / math.sqrt(32), with_lse=True)
    assert_close(out, torch.from_numpy(golden["ragged/o"]), **FWD_TOL[F16], what="ragged O")
    assert_close(lse, torch.from_numpy(golden["ragged/lse"]), **FWD_TOL[F16], what="ragged LSE")


def test_ragged_decode_with_empty_splits_and_nan_tail():
    """Sequences much shorter than the planned chunk leave whole splits empty
    (LSE -inf, weight 0); positions beyond each length hold NaN."""
    b, hkv, cap, d, hq, sq = 4, 2, 20000, 64, 8, 3
    kc = torch.full((b, hkv, cap, d), float("nan"), device="cuda", dtype=F16)
    vc = torch.full_like(kc, float("nan"))
    lengths = [1, 20000, 129, 7777]
    for i, n in enumerate(lengths):
        kc[i, :, :n] = seeded((hkv, n, d), 260 + i, dtype=F16)
        vc[i, :, :n] = seeded((hkv, n, d), 270 + i, dtype=F16)
    q = seeded((b, hq, sq, d), 280, dtype=F16)
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    out = attention_decode_ragged(q, kc, vc, lens, max_seqlen=cap, scale=0.125)
    assert torch.isfinite(out).all()
    for i, n in enumerate(lengths):
        eo, _ = reference_fp32(q[i:i + 1], kc[i:i + 1, :, :n], vc[i:i + 1, :, :n], causal=False)
        assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"seq {i}")


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("hq,hkv,q_seq,d", [
    (4, 1, 4, 64),    # 16 packed rows: one full 16-row block
    (17, 1, 1, 64),   # 17 rows: a second block with a single row
    (8, 1, 4, 128),   # 32 rows: two 16-row blocks
    (11, 1, 3, 96),   # 33 rows: four-block workgroup, partly empty
    (16, 1, 4, 64),   # 64 rows: four full blocks
    (13, 1, 5, 72),   # 65 rows: a second row block; head dim padded to 96
])
def test_decode_row_block_edges(dtype, hq, hkv, q_seq, d):
    """Packed-row counts (G * Sq) on both sides of the 16-row MFMA blocks and
    of the 16/32/64-row workgroup tiles."""
    q = seeded((2, hq, q_seq, d), 291, dtype=dtype)
    k = seeded((2, hkv, 3000, d), 292, dtype=dtype)
    v = seeded((2, hkv, 3000, d), 293, dtype=dtype)
    with torch.no_grad():
        out = attention(q, k, v, causal=False, backend="hip")
    eo, _ = reference_fp32(q, k, v, causal=False)
    assert_close(out, eo, **FWD_TOL[dtype], what="O")


@pytest.mark.parametrize("d", [64, 128])
def test_decode_merge_many_splits(d):
    """One KV group with a long cache: the planner picks 256 splits, more than
    one merge lane reads in a single round trip, so the merge walks several
    chunks with its running rescale."""
    q = seeded((1, 4, 1, d), 295, dtype=F16)
    k = seeded((1, 1, 65536, d), 296, dtype=F16)
    v = seeded((1, 1, 65536, d), 297, dtype=F16)
    assert _hip.decode_num_splits(1, 4, 1, 1, 65536, d) > 64
    out, lse = attention_forward(q, k, v, causal=False, scale=1 / math.sqrt(d))
    eo, el = reference_fp32(q, k, v, causal=False)
    assert_close(out, eo, **FWD_TOL[F16], what="O")
    assert_close(lse, el, **FWD_TOL[F16], what="LSE")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128, 72, 20])
def test_lse_merge_matches_oracle(dtype, d):
    """kf_lse_merge on partials in the reference's split layout
    (triton_forward.py:269-349) against the oracle's merge: random partials
    with empty splits (LSE = -inf) and one row whose splits are all empty."""
    from kotflash_amd.kernels.hip_decode import lse_merge
    from oracle import attention_oracle as orc

    g = torch.Generator().manual_seed(940 + d)
    ns, b, h, sq = 37, 2, 3, 5
    part_o = torch.randn(ns, b, h, sq, d, generator=g)
    part_lse = torch.randn(ns, b, h, sq, generator=g) * 4
    part_lse[3] = float("-inf")                 # an empty split for every row
    part_lse[:, 1, 2, 4] = float("-inf")        # a row with no visible key at all
    part_o[:, 1, 2, 4] = 0.0
    out, lse = lse_merge(part_o.cuda(), part_lse.cuda(), dtype=dtype)
    eo, el = orc.split_kv_merge(part_o.numpy(), part_lse.numpy())
    assert out.dtype == dtype and lse.shape == (b, h, sq)
    assert_close(out, torch.from_numpy(eo), **FWD_TOL[dtype], what="merged O")
    finite = torch.ones(b, h, sq, dtype=torch.bool)
    finite[1, 2, 4] = False
    assert_close(lse.cpu()[finite], torch.from_numpy(el)[finite], atol=1e-5, rtol=1e-5,
                 what="merged LSE")
    assert torch.isneginf(lse[1, 2, 4]) and (out[1, 2, 4] == 0).all()


def test_lse_merge_of_oracle_split_partials_is_full_attention():
    """Partials from the oracle's split kernel (uneven chunks, a ragged
    sequence whose later splits are empty) merged on the GPU equal dense
    attention: the merge is exact up to the output rounding."""
    from kotflash_amd.kernels.hip_decode import lse_merge
    from oracle import attention_oracle as orc

    q = seeded((2, 8, 3, 64), 950, dtype=F16)
    k = seeded((2, 2, 1500, 64), 951, dtype=F16)
    v = seeded((2, 2, 1500, 64), 952, dtype=F16)
    lengths = [1500, 700]
    n = lambda t: t.cpu().float().numpy()
    po, pl = orc.split_kv_partials(n(q), n(k), n(v), scale=0.125, num_splits=6, chunk_n=256,
                                   seqlens=lengths)
    out, lse = lse_merge(torch.from_numpy(po).float().cuda(), torch.from_numpy(pl).float().cuda())
    for i, L in enumerate(lengths):
        eo, el = reference_fp32(q[i:i + 1], k[i:i + 1, :, :L], v[i:i + 1, :, :L], causal=False,
                                scale=0.125)
        assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"O seq {i}")
        assert_close(lse[i:i + 1], el, atol=1e-4, rtol=1e-5, what=f"LSE seq {i}")


def test_validated_decode_check_agrees_with_the_full_one():
    """The public ``attention``'s decode lane checks only what its validation
    left open; on validated inputs it must decide as ``strided_decode_supported``."""
    from kotflash_amd.kernels.hip_decode import strided_decode_supported, validated_decode_supported

    cases = []
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        for sq, sk, d in ((1, 4096, 64), (16, 1024, 128), (17, 4096, 64), (1, 1023, 64),
                          (1, 2048, 72), (1, 2048, 20), (4, 2048, 136)):
            q = torch.zeros((2, 8, sq, d), device="cuda", dtype=dtype)
            k = torch.zeros((2, 2, sk, d), device="cuda", dtype=dtype)
            cases.append((q, k, k.clone()))
    base = torch.zeros((2, 2, 4096 + 64, 64), device="cuda", dtype=torch.float16)
    cases.append((torch.zeros((2, 8, 1, 64), device="cuda", dtype=torch.float16),
                  base[:, :, :3000], base[:, :, :3000]))              # padded cache view
    wide = torch.zeros((2, 2, 2048, 72), device="cuda", dtype=torch.float16)[..., :64]
    cases.append((torch.zeros((2, 8, 1, 64), device="cuda", dtype=torch.float16), wide, wide))
    odd = torch.zeros((2 * 2 * 2048 * 64 + 4,), device="cuda", dtype=torch.float16)[4:].view(2, 2, 2048, 64)
    cases.append((torch.zeros((2, 8, 1, 64), device="cuda", dtype=torch.float16), odd, odd))
    seen = set()
    for q, k, v in cases:
        full, lean = strided_decode_supported(q, k, v), validated_decode_supported(q, k, v)
        assert full == lean, (tuple(q.shape), tuple(k.shape), k.stride(), q.dtype)
        seen.add(full)
    assert seen == {True, False}


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_long_context_decode(dtype):
    """A 256K-key cache (D=128, MQA with 16 query heads, 4 new tokens per
    sequence): the split plan's largest chunks, per-head K/V slices of
    64 MiB and the merge of many splits, against dense fp32 attention, and
    the public API on a padded view of a longer cache."""
    sk, d = 262144, 128
    q = seeded((1, 16, 4, d), 1801, dtype=dtype)
    k = seeded((1, 1, sk, d), 1802, dtype=dtype)
    v = seeded((1, 1, sk, d), 1803, dtype=dtype)
    out, lse = attention_forward(q, k, v, causal=False, scale=1 / math.sqrt(d))
    eo, el = reference_fp32(q, k, v, causal=False)
    assert_close(out, eo, **FWD_TOL[dtype], what="O")
    assert_close(lse, el, **FWD_TOL[dtype], what="LSE")
    big_k = torch.zeros((1, 1, sk + 1000, d), device="cuda", dtype=dtype)
    big_v = torch.full((1, 1, sk + 1000, d), float("nan"), device="cuda", dtype=dtype)
    big_k[:, :, :sk] = k
    big_v[:, :, :sk] = v
    out2 = attention(q, big_k[:, :, :sk], big_v[:, :, :sk], causal=False, backend="hip")
    assert torch.equal(out, out2)
