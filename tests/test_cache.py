"""CPU behaviour of the cache API (the reference's tests/test_kv_cache.py and
tests/test_preallocated_cache.py contract, plus the ragged extension)."""
import pytest
import torch
import torch.nn.functional as F

from kotflash_amd.cache import (
    PreallocatedKVCache, RaggedKVCache, append_kv_cache, decode_step,
)


def test_append_kv_cache_preserves_order_and_inputs():
    k_cache = torch.arange(24, dtype=torch.float32).view(1, 2, 3, 4)
    v_cache = -k_cache
    new_k = torch.full((1, 2, 1, 4), 100.0)
    new_v = -new_k
    old_k, old_v = k_cache.clone(), v_cache.clone()
    uk, uv = append_kv_cache(k_cache, v_cache, new_k, new_v)
    torch.testing.assert_close(uk, torch.cat((old_k, new_k), 2))
    torch.testing.assert_close(uv, torch.cat((old_v, new_v), 2))
    torch.testing.assert_close(k_cache, old_k)
    torch.testing.assert_close(v_cache, old_v)


@pytest.mark.parametrize("bad", ["batch", "heads", "dim", "dtype"])
def test_append_kv_cache_rejects_incompatible(bad):
    kc = torch.zeros(1, 2, 4, 8)
    nk = {"batch": torch.zeros(2, 2, 1, 8), "heads": torch.zeros(1, 1, 1, 8),
          "dim": torch.zeros(1, 2, 1, 16), "dtype": torch.zeros(1, 2, 1, 8).half()}[bad]
    with pytest.raises(ValueError):
        append_kv_cache(kc, kc.clone(), nk, nk.clone())


def test_append_kv_cache_rejects_zero_heads():
    empty = torch.empty(1, 0, 2, 8)
    with pytest.raises(ValueError, match="non-zero"):
        append_kv_cache(empty, empty, torch.empty(1, 0, 1, 8), torch.empty(1, 0, 1, 8))


def test_decode_step_matches_expanded_sdpa():
    torch.manual_seed(7)
    q = torch.randn(1, 4, 1, 16)
    kc = torch.randn(1, 2, 5, 16)
    vc = torch.randn_like(kc)
    kn = torch.randn(1, 2, 1, 16)
    vn = torch.randn_like(kn)
    out, uk, uv = decode_step(q, kc, vc, kn, vn, backend="sdpa")
    expected = F.scaled_dot_product_attention(q, uk.repeat_interleave(2, 1), uv.repeat_interleave(2, 1))
    torch.testing.assert_close(out, expected)
    assert uk.shape[2] == uv.shape[2] == 6


def test_decode_step_rejections():
    cache = torch.randn(1, 2, 4, 16)
    new = torch.randn(1, 2, 1, 16)
    with pytest.raises(ValueError, match="exactly one new query token"):
        decode_step(torch.randn(1, 4, 2, 16), cache, cache, new, new, backend="sdpa")
    with pytest.raises(ValueError, match="divisible"):
        decode_step(torch.randn(1, 3, 1, 16), cache, cache, new, new, backend="sdpa")
    with pytest.raises(ValueError, match="exactly one new K/V token"):
        decode_step(torch.randn(1, 4, 1, 16), cache, cache, torch.randn(1, 2, 2, 16),
                    torch.randn(1, 2, 2, 16), backend="sdpa")


def test_preallocated_cache_prefix_views_share_storage():
    cache = PreallocatedKVCache(1, 2, 8, 4, device="cpu", dtype=torch.float32)
    k1 = torch.arange(24, dtype=torch.float32).view(1, 2, 3, 4)
    k2 = torch.full((1, 2, 1, 4), 100.0)
    cache.append(k1, -k1)
    cache.append(k2, -k2)
    assert cache.length == 4
    vk, vv = cache.view()
    torch.testing.assert_close(vk, torch.cat((k1, k2), 2))
    torch.testing.assert_close(vv, -torch.cat((k1, k2), 2))
    assert vk.untyped_storage().data_ptr() == cache.k.untyped_storage().data_ptr()
    ck, cv = cache.contiguous_view()
    assert ck.is_contiguous() and cv.is_contiguous()
    torch.testing.assert_close(ck, vk)


def test_preallocated_cache_hides_unused_slots():
    cache = PreallocatedKVCache(1, 1, 5, 4, device="cpu", dtype=torch.float32)
    cache.k.fill_(12345.0)
    cache.v.fill_(-12345.0)
    k = torch.ones(1, 1, 2, 4)
    cache.append(k, 2 * k)
    ak, av = cache.view()
    assert ak.shape[2] == av.shape[2] == 2
    torch.testing.assert_close(ak, k)
    torch.testing.assert_close(av, 2 * k)
    assert (cache.k[:, :, 2:] == 12345.0).all()


def test_preallocated_cache_rejects_without_advancing():
    cache = PreallocatedKVCache(1, 2, 3, 4, device="cpu", dtype=torch.float32)
    with pytest.raises(ValueError, match="empty"):
        cache.view()
    with pytest.raises(ValueError, match="batch, heads"):
        cache.append(torch.zeros(1, 1, 1, 4), torch.zeros(1, 1, 1, 4))
    with pytest.raises(ValueError, match="dtype"):
        cache.append(torch.zeros(1, 2, 1, 4).half(), torch.zeros(1, 2, 1, 4).half())
    with pytest.raises(ValueError, match="shapes must match"):
        cache.append(torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 2, 4))
    with pytest.raises(ValueError, match="backend"):
        cache.append(torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 1, 4), backend="bogus")
    assert cache.length == 0
    cache.append(torch.zeros(1, 2, 2, 4), torch.zeros(1, 2, 2, 4))
    with pytest.raises(ValueError, match="full"):
        cache.append(torch.zeros(1, 2, 2, 4), torch.zeros(1, 2, 2, 4))
    assert cache.length == 2


@pytest.mark.parametrize("bad", [0, -1, 1.5, True])
def test_preallocated_cache_rejects_bad_dims(bad):
    with pytest.raises(ValueError, match="positive integer"):
        PreallocatedKVCache(1, 2, bad, 4, device="cpu", dtype=torch.float32)


def test_preallocated_cache_attend_and_append_and_attend():
    torch.manual_seed(21)
    cache = PreallocatedKVCache(1, 2, 16, 16, device="cpu", dtype=torch.float32)
    pk, pv = torch.randn(1, 2, 5, 16), torch.randn(1, 2, 5, 16)
    nk, nv = torch.randn(1, 2, 1, 16), torch.randn(1, 2, 1, 16)
    q = torch.randn(1, 4, 1, 16)
    cache.append(pk, pv)
    out = cache.attend(q, backend="sdpa")
    torch.testing.assert_close(out, F.scaled_dot_product_attention(
        q, pk.repeat_interleave(2, 1), pv.repeat_interleave(2, 1)))
    out2 = cache.append_and_attend(q, nk, nv, append_backend="torch", attention_backend="sdpa")
    torch.testing.assert_close(out2, F.scaled_dot_product_attention(
        q, torch.cat((pk, nk), 2).repeat_interleave(2, 1), torch.cat((pv, nv), 2).repeat_interleave(2, 1)))
    assert cache.length == 6
    with pytest.raises(ValueError, match="requires attention_backend"):
        cache.append_and_attend(q, nk, nv, append_backend="fused", attention_backend="sdpa")
    assert cache.length == 6


def test_ragged_cache_appends_each_sequence_at_its_length():
    cache = RaggedKVCache(3, 1, 10, 4, device="cpu", dtype=torch.float32)
    cache.k.fill_(-7.0)
    cache.set_lengths([0, 4, 7])
    new = torch.arange(3 * 2 * 4, dtype=torch.float32).view(3, 1, 2, 4)
    cache.append(new, -new, backend="torch")
    assert cache.lengths == [2, 6, 9]
    for b, start in enumerate([0, 4, 7]):
        torch.testing.assert_close(cache.k[b, :, start:start + 2], new[b])
        torch.testing.assert_close(cache.v[b, :, start:start + 2], -new[b])
    assert (cache.k[0, :, 2:] == -7).all() and (cache.k[1, :, 6:] == -7).all()
    with pytest.raises(ValueError, match="full"):
        cache.append(new, new, backend="torch")
    assert cache.lengths == [2, 6, 9]
    assert cache.seqlens.tolist() == [2, 6, 9] and cache.starts.tolist() == [2, 6, 9]


def test_ragged_cache_attend_matches_per_sequence_sdpa():
    torch.manual_seed(5)
    cache = RaggedKVCache(2, 2, 12, 8, device="cpu", dtype=torch.float32)
    cache.k.normal_()
    cache.v.normal_()
    cache.set_lengths([3, 12])
    q = torch.randn(2, 4, 2, 8)
    out = cache.attend(q, backend="sdpa")
    for b, n in enumerate([3, 12]):
        exp = F.scaled_dot_product_attention(
            q[b:b + 1], cache.k[b:b + 1, :, :n].repeat_interleave(2, 1),
            cache.v[b:b + 1, :, :n].repeat_interleave(2, 1))
        torch.testing.assert_close(out[b:b + 1], exp)
    with pytest.raises(ValueError, match="lengths"):
        cache.set_lengths([1, 13])


def test_ragged_cache_append_and_attend_two_step_path_on_cpu():
    """On the CPU, append_and_attend appends with torch copies and attends per
    sequence with SDPA; the fused path is GPU-only and refuses SDPA, and a
    rejected append leaves lengths and storage untouched."""
    torch.manual_seed(6)
    cache = RaggedKVCache(2, 1, 9, 8, device="cpu", dtype=torch.float32)
    cache.k.normal_()
    cache.v.normal_()
    cache.set_lengths([2, 5])
    nk, nv = torch.randn(2, 1, 3, 8), torch.randn(2, 1, 3, 8)
    q = torch.randn(2, 2, 3, 8)
    out = cache.append_and_attend(q, nk, nv)
    assert cache.lengths == [5, 8]
    for b, n in enumerate([5, 8]):
        torch.testing.assert_close(cache.k[b, :, n - 3:n], nk[b])
        exp = F.scaled_dot_product_attention(
            q[b:b + 1], cache.k[b:b + 1, :, :n].repeat_interleave(2, 1),
            cache.v[b:b + 1, :, :n].repeat_interleave(2, 1))
        torch.testing.assert_close(out[b:b + 1], exp)
    before = cache.k.clone()
    with pytest.raises(ValueError, match="full"):
        cache.append_and_attend(q, nk, nv)
    assert cache.lengths == [5, 8] and torch.equal(cache.k, before)
    with pytest.raises(ValueError, match="fused"):
        cache.append_and_attend(q[:, :, :1], nk[:, :, :1], nv[:, :, :1], append_backend="fused",
                                attention_backend="sdpa")
    with pytest.raises(ValueError, match="append backend"):
        cache.append_and_attend(q, nk, nv, append_backend="nope")


def test_auto_fuses_routing(monkeypatch):
    """append_backend='auto' picks the fused append + decode only for
    inference-only calls whose attention goes to the HIP decode; the native
    append check (_use_hip_append) is patched in, so this runs on the CPU."""
    from kotflash_amd import cache as cache_mod

    monkeypatch.setattr(cache_mod, "_use_hip_append", lambda backend, t: True)
    kc = torch.empty(2, 2, 8, 64, dtype=torch.float16)
    q = torch.empty(2, 8, 1, 64, dtype=torch.float16)
    fuses = cache_mod._auto_fuses
    assert fuses(q, kc, 4096, "auto", False)            # split-KV decode shape
    assert fuses(q, kc, 100, "auto", False)             # auto inference -> HIP at any size
    assert fuses(q, kc, 100, "hip", False)              # HIP forced
    assert not fuses(q, kc, 4096, "sdpa", False)
    assert not fuses(q, kc, 4096, "auto", True)         # autograd
    q72 = torch.empty(2, 8, 1, 12, dtype=torch.float16)
    assert not fuses(q72, torch.empty(2, 2, 8, 12, dtype=torch.float16), 4096, "hip", False)
    assert not fuses(q.float(), kc.float(), 4096, "auto", False)  # fp32: SDPA
    monkeypatch.setattr(cache_mod, "_use_hip_append", lambda backend, t: False)
    assert not fuses(q, kc, 4096, "hip", False)         # native append disabled
