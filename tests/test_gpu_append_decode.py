"""Fused append + split-KV decode (kf_attn_append_decode) on the GPU.

One decode launch stores the new tokens into the cache and attends over the
old keys plus the new ones (reference kotflash/kernels/triton_decode.py:
302-386 folds one token's slot write into its split kernel the same way).
Checked here:
- the cache after the call equals slice assignment, bit for bit, with every
  other slot (NaN sentinels) untouched;
- O and LSE against dense fp32 attention over each sequence's first
  L_b + n positions (fp16 atol = rtol = 2e-3, bf16 1e-2);
- ragged lengths including 0, granule boundaries (127, 128, 129) and a
  sequence that fills the cache to capacity; n in 1..16, Sq = 1 and Sq = n;
- the scalar entry (attention_forward_strided_append) and the cache classes.
"""
import pytest
import torch

from kotflash_amd.cache import RaggedKVCache
from kotflash_amd.kernels.hip_decode import (attention_append_decode_ragged,
                                             attention_decode_ragged,
                                             attention_forward_strided_append)
from tests.gpu_helpers import FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


def _nan_cache(b, hkv, cap, d, dtype, lengths, seed):
    kc = torch.full((b, hkv, cap, d), float("nan"), device="cuda", dtype=dtype)
    vc = torch.full_like(kc, float("nan"))
    for i, n in enumerate(lengths):
        if n:
            kc[i, :, :n] = seeded((hkv, n, d), seed + 2 * i, dtype=dtype)
            vc[i, :, :n] = seeded((hkv, n, d), seed + 2 * i + 1, dtype=dtype)
    return kc, vc


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n,sq", [(1, 1), (5, 5), (16, 16), (16, 1)])
def test_ragged_append_decode(dtype, d, n, sq):
    b, hkv, hq, cap = 6, 2, 8, 2048
    lengths = [0, 127, 128, 129, 1500, cap - n]
    kc, vc = _nan_cache(b, hkv, cap, d, dtype, lengths, 9100)
    nk = seeded((b, hkv, n, d), 9200, dtype=dtype)
    nv = seeded((b, hkv, n, d), 9201, dtype=dtype)
    q = seeded((b, hq, sq, d), 9202, dtype=dtype)
    ek, ev = kc.clone(), vc.clone()
    for i, s in enumerate(lengths):
        ek[i, :, s:s + n] = nk[i]
        ev[i, :, s:s + n] = nv[i]
    seqlens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    print(f"ragged append+decode dtype={dtype} d={d} n={n} sq={sq}", flush=True)
    out, lse = attention_append_decode_ragged(q, kc, vc, nk, nv, seqlens, host_lengths=lengths,
                                              scale=d ** -0.5, with_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(_bits(kc), _bits(ek)) and torch.equal(_bits(vc), _bits(ev))
    tol = FWD_TOL[dtype]
    for i, s in enumerate(lengths):
        eo, el = reference_fp32(q[i:i + 1], ek[i:i + 1, :, :s + n], ev[i:i + 1, :, :s + n],
                                causal=False)
        assert_close(out[i:i + 1], eo, **tol, what=f"O seq {i} (L={s})")
        assert_close(lse[i:i + 1], el, **tol, what=f"LSE seq {i} (L={s})")


def test_ragged_append_decode_empty_cache_and_agrees_with_two_step_path():
    """All lengths 0 (only the new tokens are visible), then a second call on
    the grown cache compared with append + ragged decode on a copy."""
    b, hkv, hq, cap, d, n = 2, 4, 16, 512, 64, 3
    kc, vc = _nan_cache(b, hkv, cap, d, F16, [0, 0], 9300)
    nk = seeded((b, hkv, n, d), 9301, dtype=F16)
    nv = seeded((b, hkv, n, d), 9302, dtype=F16)
    q = seeded((b, hq, n, d), 9303, dtype=F16)
    seqlens = torch.zeros(b, device="cuda", dtype=torch.int32)
    out = attention_append_decode_ragged(q, kc, vc, nk, nv, seqlens, host_lengths=[0, 0],
                                         scale=0.125)
    eo, _ = reference_fp32(q, nk, nv, causal=False)
    assert_close(out, eo, **FWD_TOL[F16], what="O over new tokens only")
    assert torch.equal(kc[:, :, :n], nk) and torch.equal(vc[:, :, :n], nv)
    assert torch.isnan(kc[:, :, n:]).all() and torch.isnan(vc[:, :, n:]).all()

    lengths = [n, n]
    nk2 = seeded((b, hkv, 2, d), 9304, dtype=F16)
    nv2 = seeded((b, hkv, 2, d), 9305, dtype=F16)
    q2 = seeded((b, hq, 1, d), 9306, dtype=F16)
    kc2, vc2 = kc.clone(), vc.clone()
    seqlens.fill_(n)
    fused = attention_append_decode_ragged(q2, kc, vc, nk2, nv2, seqlens,
                                           host_lengths=lengths, scale=0.125)
    kc2[:, :, n:n + 2] = nk2
    vc2[:, :, n:n + 2] = nv2
    seq2 = torch.full((b,), n + 2, device="cuda", dtype=torch.int32)
    two_step = attention_decode_ragged(q2, kc2, vc2, seq2, max_seqlen=n + 2, scale=0.125)
    assert torch.equal(_bits(kc), _bits(kc2)) and torch.equal(_bits(vc), _bits(vc2))
    assert_close(fused, two_step, **FWD_TOL[F16], what="fused vs two-step")


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("past", [0, 1, 1023, 4095])
def test_strided_append_scalar_position(dtype, past):
    b, hkv, hq, cap, d = 2, 2, 8, 4096, 64
    kc, vc = _nan_cache(b, hkv, cap, d, dtype, [past] * b, 9400)
    nk = seeded((b, hkv, 1, d), 9401, dtype=dtype)
    nv = seeded((b, hkv, 1, d), 9402, dtype=dtype)
    q = seeded((b, hq, 1, d), 9403, dtype=dtype)
    print(f"strided append dtype={dtype} past={past}", flush=True)
    out = attention_forward_strided_append(q, kc, vc, nk, nv, past_length=past, scale=0.125)
    torch.cuda.synchronize()
    assert torch.equal(kc[:, :, past:past + 1], nk) and torch.equal(vc[:, :, past:past + 1], nv)
    assert torch.isnan(kc[:, :, past + 1:]).all() and torch.isnan(vc[:, :, past + 1:]).all()
    eo, _ = reference_fp32(q, kc[:, :, :past + 1], vc[:, :, :past + 1], causal=False)
    assert_close(out, eo, **FWD_TOL[dtype], what=f"O past={past}")


def test_ragged_cache_append_and_attend_fused_config5_steps():
    """BASELINE config 5 shape for 6 steps through RaggedKVCache.append_and_attend
    (auto = fused): cache [8, 8, 32768, 64] fp16, lengths U[4096, 28000],
    n in [1, 16], Hq = 32 queries per new token."""
    g = torch.Generator().manual_seed(501)
    b, hkv, cap, d, hq = 8, 8, 32768, 64, 32
    cache = RaggedKVCache(b, hkv, cap, d, device="cuda", dtype=F16)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    lengths = torch.randint(4096, 28001, (b,), generator=g).tolist()
    for i, n in enumerate(lengths):
        cache.k[i, :, :n] = seeded((hkv, n, d), 530 + i, dtype=F16)
        cache.v[i, :, :n] = seeded((hkv, n, d), 540 + i, dtype=F16)
    cache.set_lengths(lengths)
    for step in range(6):
        n = int(torch.randint(1, 17, (1,), generator=g))
        nk = seeded((b, hkv, n, d), 610 + step, dtype=F16)
        nv = seeded((b, hkv, n, d), 710 + step, dtype=F16)
        q = seeded((b, hq, n, d), 810 + step, dtype=F16)
        before = list(cache.lengths)
        with torch.inference_mode():
            out = cache.append_and_attend(q, nk, nv)
        assert cache.lengths == [x + n for x in before]
        for i, s in enumerate(before):
            assert torch.equal(cache.k[i, :, s:s + n], nk[i])
            assert torch.equal(cache.v[i, :, s:s + n], nv[i])
            assert torch.isnan(cache.k[i, :, s + n:s + n + 16]).all()
        assert torch.isfinite(out).all()
        for i in (0, step % b, b - 1):
            kv, vv = cache.view(i)
            eo, _ = reference_fp32(q[i:i + 1], kv, vv, causal=False)
            assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"step {step} seq {i}")


def test_fused_matches_oracle_append_then_split_merge():
    """The fused call against the CPU oracle's own composition: kv_append
    (kv_append_cuda.cu:12-40, per-sequence starts), then split-KV partials
    over the post-append lengths and the LSE merge (triton_forward.py:
    169-349). Cache bit-exact; O and LSE to fp16 tolerance."""
    import numpy as np

    from oracle import attention_oracle as orc

    b, hkv, hq, cap, d, n = 3, 2, 8, 640, 64, 4
    lengths = [0, 200, 500]
    kc, vc = _nan_cache(b, hkv, cap, d, F16, lengths, 9500)
    nk = seeded((b, hkv, n, d), 9501, dtype=F16)
    nv = seeded((b, hkv, n, d), 9502, dtype=F16)
    q = seeded((b, hq, n, d), 9503, dtype=F16)
    ek, ev = kc.cpu().numpy(), vc.cpu().numpy()
    orc.kv_append(ek, ev, nk.cpu().numpy(), nv.cpu().numpy(), lengths)
    seqlens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    out, lse = attention_append_decode_ragged(q, kc, vc, nk, nv, seqlens, host_lengths=lengths,
                                              scale=0.125, with_lse=True)
    assert kc.cpu().numpy().view(np.int16).tobytes() == ek.view(np.int16).tobytes()
    assert vc.cpu().numpy().view(np.int16).tobytes() == ev.view(np.int16).tobytes()
    after = [x + n for x in lengths]
    po, pl = orc.split_kv_partials(q.cpu().numpy(), np.nan_to_num(ek), np.nan_to_num(ev),
                                   scale=0.125, num_splits=3, chunk_n=256, seqlens=after)
    eo, el = orc.split_kv_merge(po, pl)
    assert_close(out, torch.from_numpy(eo), **FWD_TOL[F16], what="O vs oracle")
    assert_close(lse, torch.from_numpy(el), **FWD_TOL[F16], what="LSE vs oracle")


@pytest.mark.parametrize("n", [33, 200])
def test_ragged_append_decode_many_new_tokens(n):
    """More new tokens than one 32-key step: the new-token split streams
    several steps over all four waves (keys 32 w + 128 j) before its copy."""
    b, hkv, hq, cap, d = 3, 2, 4, 1024, 128
    lengths = [0, 300, cap - n]
    kc, vc = _nan_cache(b, hkv, cap, d, F16, lengths, 9600)
    nk = seeded((b, hkv, n, d), 9601, dtype=F16)
    nv = seeded((b, hkv, n, d), 9602, dtype=F16)
    q = seeded((b, hq, 2, d), 9603, dtype=F16)
    seqlens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    print(f"ragged append+decode n={n}", flush=True)
    out = attention_append_decode_ragged(q, kc, vc, nk, nv, seqlens, host_lengths=lengths,
                                         scale=d ** -0.5)
    torch.cuda.synchronize()
    for i, s in enumerate(lengths):
        assert torch.equal(kc[i, :, s:s + n], nk[i]) and torch.equal(vc[i, :, s:s + n], nv[i])
        assert torch.isnan(kc[i, :, s + n:]).all() and torch.isnan(kc[i, :, :s]).logical_not().all()
        eo, _ = reference_fp32(q[i:i + 1], kc[i:i + 1, :, :s + n], vc[i:i + 1, :, :s + n],
                               causal=False)
        assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"O seq {i} (L={s}, n={n})")


def test_preallocated_cache_auto_takes_fused_path_when_it_applies(monkeypatch):
    """PreallocatedKVCache.append_and_attend with the default backends fuses
    the append into the decode for inference-only calls (auto sends
    inference to the HIP kernels at any cache length), and keeps the two-step
    path with autograd."""
    from kotflash_amd.cache import PreallocatedKVCache
    import kotflash_amd.kernels.hip_decode as hd

    calls = []
    real = hd.attention_forward_strided_append

    def counting(*args, **kwargs):
        calls.append(kwargs["past_length"])
        return real(*args, **kwargs)

    monkeypatch.setattr(hd, "attention_forward_strided_append", counting)
    cache = PreallocatedKVCache(2, 2, 4096, 64, device="cuda", dtype=F16)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    pk, pv = seeded((2, 2, 2047, 64), 9701, dtype=F16), seeded((2, 2, 2047, 64), 9702, dtype=F16)
    cache.append(pk, pv, backend="torch")
    nk, nv = seeded((2, 2, 1, 64), 9703, dtype=F16), seeded((2, 2, 1, 64), 9704, dtype=F16)
    q = seeded((2, 8, 1, 64), 9705, dtype=F16)
    with torch.inference_mode():
        out = cache.append_and_attend(q, nk, nv)
    assert calls == [2047] and cache.length == 2048
    assert torch.equal(cache.k[:, :, 2047:2048], nk) and torch.isnan(cache.k[:, :, 2048:]).all()
    eo, _ = reference_fp32(q, torch.cat((pk, nk), 2), torch.cat((pv, nv), 2), causal=False)
    assert_close(out, eo, **FWD_TOL[F16], what="auto (fused) O")
    # Autograd: the two-step path.
    qg = q.clone().requires_grad_(True)
    out2 = cache.append_and_attend(qg, nk, nv)
    assert calls == [2047] and cache.length == 2049 and out2.requires_grad
    # A cache below the split-KV decode envelope fuses too (inference).
    small = PreallocatedKVCache(2, 2, 256, 64, device="cuda", dtype=F16)
    small.append(pk[:, :, :100], pv[:, :, :100], backend="torch")
    with torch.inference_mode():
        out3 = small.append_and_attend(q, nk, nv)
    assert calls == [2047, 100] and small.length == 101
    assert torch.equal(small.k[:, :, 100:101], nk)
    eo, _ = reference_fp32(q, torch.cat((pk[:, :, :100], nk), 2),
                           torch.cat((pv[:, :, :100], nv), 2), causal=False)
    assert_close(out3, eo, **FWD_TOL[F16], what="auto (fused, short cache) O")
