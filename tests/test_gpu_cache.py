"""K/V append on the GPU (through the C ABI): bit-exact against slice
assignment, per-sequence positions, strided sources, untouched slots, and the
BASELINE config 5 append + ragged decode loop."""
import pytest
import torch

from kotflash_amd._hip_append import append_kv_cuda, append_kv_hip
from kotflash_amd.cache import PreallocatedKVCache, RaggedKVCache
from tests.gpu_helpers import FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


def test_append_matches_golden(golden):
    kc = torch.from_numpy(golden["append/k_cache"]).cuda()
    vc = torch.from_numpy(golden["append/v_cache"]).cuda()
    nk = torch.from_numpy(golden["append/new_k"]).cuda()
    nv = torch.from_numpy(golden["append/new_v"]).cuda()
    starts = torch.from_numpy(golden["append/starts"]).cuda()
    append_kv_hip(kc, vc, nk, nv, starts)
    assert kc.cpu().numpy().tobytes() == golden["append/k_expected"].tobytes()
    assert vc.cpu().numpy().tobytes() == golden["append/v_expected"].tobytes()


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("d", [8, 64, 72, 128, 12])
def test_append_bit_exact_scalar_start(dtype, d):
    kc = torch.full((2, 3, 50, d), float("nan"), device="cuda", dtype=dtype)
    vc = torch.full_like(kc, float("nan"))
    nk = seeded((2, 3, 7, d), 301, dtype=dtype)
    nv = seeded((2, 3, 7, d), 302, dtype=dtype)
    ek, ev = kc.clone(), vc.clone()
    ek[:, :, 40:47] = nk
    ev[:, :, 40:47] = nv
    append_kv_hip(kc, vc, nk, nv, 40)
    # NaN-aware bitwise equality: compare raw bits.
    assert torch.equal(kc.view(torch.int16), ek.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), ev.view(torch.int16))


def test_append_strided_sources_and_per_sequence_starts():
    base_k = seeded((4, 5, 2, 64), 311, dtype=F16)  # [B, S, H, D] storage
    base_v = seeded((4, 5, 2, 64), 312, dtype=F16)
    nk, nv = base_k.transpose(1, 2), base_v.transpose(1, 2)  # [B, H, S, D] views
    assert not nk.is_contiguous()
    kc = torch.zeros((4, 2, 30, 64), device="cuda", dtype=F16)
    vc = torch.zeros_like(kc)
    starts = [0, 25, 3, 11]
    append_kv_hip(kc, vc, nk, nv, torch.tensor(starts, device="cuda"))
    ek, ev = torch.zeros_like(kc), torch.zeros_like(vc)
    for b, s in enumerate(starts):
        ek[b, :, s:s + 5] = nk[b]
        ev[b, :, s:s + 5] = nv[b]
    assert torch.equal(kc, ek) and torch.equal(vc, ev)
    # Element-wise path: non-unit head_dim stride in the source.
    odd = seeded((1, 2, 3, 128), 313, dtype=F16)[..., ::2]
    kc2 = torch.zeros((1, 2, 8, 64), device="cuda", dtype=F16)
    vc2 = torch.zeros_like(kc2)
    append_kv_cuda(kc2, vc2, odd, odd, 2)
    assert torch.equal(kc2[:, :, 2:5], odd) and (kc2[:, :, :2] == 0).all()


def test_append_rejects_before_writing():
    kc = torch.zeros((1, 2, 8, 64), device="cuda", dtype=F16)
    nk = torch.ones((1, 2, 3, 64), device="cuda", dtype=F16)
    with pytest.raises(RuntimeError, match="capacity"):
        append_kv_hip(kc, kc.clone(), nk, nk, 6)
    with pytest.raises(TypeError):
        append_kv_hip(kc.float(), kc.float(), nk.float(), nk.float(), 0)
    assert (kc == 0).all()


def test_preallocated_cache_hip_append():
    """The reference's CUDA-append case (tests/test_cuda_append.py:18-34)."""
    cache = PreallocatedKVCache(2, 2, 64, 32, device="cuda", dtype=F16)
    pk, pv = seeded((2, 2, 7, 32), 321, dtype=F16), seeded((2, 2, 7, 32), 322, dtype=F16)
    nk, nv = seeded((2, 2, 3, 32), 323, dtype=F16), seeded((2, 2, 3, 32), 324, dtype=F16)
    cache.append(pk, pv, backend="cuda")
    cache.append(nk, nv, backend="hip")
    ak, av = cache.view()
    assert torch.equal(ak, torch.cat((pk, nk), 2)) and torch.equal(av, torch.cat((pv, nv), 2))
    assert cache.length == 10


def test_config5_append_and_ragged_decode_steps():
    """BASELINE config 5, shortened to 6 steps: cache [8, 8, 32768, 64] fp16,
    per-sequence lengths U[4096, 28000], unused capacity NaN; each step appends
    n in [1, 16] tokens per sequence (bit-exact check) and decodes Hq=32 rows
    per sequence over its visible prefix."""
    g = torch.Generator().manual_seed(500)
    b, hkv, cap, d, hq = 8, 8, 32768, 64, 32
    cache = RaggedKVCache(b, hkv, cap, d, device="cuda", dtype=F16)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    lengths = torch.randint(4096, 28001, (b,), generator=g).tolist()
    for i, n in enumerate(lengths):
        cache.k[i, :, :n] = seeded((hkv, n, d), 510 + i, dtype=F16)
        cache.v[i, :, :n] = seeded((hkv, n, d), 520 + i, dtype=F16)
    cache.set_lengths(lengths)
    for step in range(6):
        n = int(torch.randint(1, 17, (1,), generator=g))
        nk = seeded((b, hkv, n, d), 600 + step, dtype=F16)
        nv = seeded((b, hkv, n, d), 700 + step, dtype=F16)
        before = list(cache.lengths)
        cache.append(nk, nv, backend="hip")
        for i, s in enumerate(before):
            assert torch.equal(cache.k[i, :, s:s + n], nk[i])
            assert torch.equal(cache.v[i, :, s:s + n], nv[i])
        q = seeded((b, hq, n, d), 800 + step, dtype=F16)
        out = cache.attend(q, backend="hip")
        assert torch.isfinite(out).all()
        for i in (0, step % b, b - 1):
            kv, vv = cache.view(i)
            eo, _ = reference_fp32(q[i:i + 1], kv, vv, causal=False)
            assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"step {step} seq {i}")


def test_device_start_out_of_range_raises_before_writing():
    """A per-sequence device start that would write past the capacity (or
    below 0) is rejected before any launch, as the reference rejects a bad
    scalar start (kv_append_cuda.cu:72-73); the caches stay unchanged."""
    kc = torch.zeros((3, 2, 16, 64), device="cuda", dtype=F16)
    vc = torch.zeros_like(kc)
    nk = torch.ones((3, 2, 4, 64), device="cuda", dtype=F16)
    for bad in ([0, 13, 2], [0, -1, 2]):
        starts = torch.tensor(bad, device="cuda")
        with pytest.raises(RuntimeError, match="capacity"):
            append_kv_hip(kc, vc, nk, nk, starts)                      # checked via a host copy
        with pytest.raises(RuntimeError, match="capacity"):
            append_kv_hip(kc, vc, nk, nk, starts, host_starts=bad)     # checked via the mirror
    torch.cuda.synchronize()
    assert (kc == 0).all() and (vc == 0).all()
    with pytest.raises(ValueError, match="one entry per batch"):
        append_kv_hip(kc, vc, nk, nk, torch.zeros(3, device="cuda", dtype=torch.int64),
                      host_starts=[0, 0])


def test_c_abi_rejects_out_of_range_device_positions():
    """Through the C ABI alone (no Python-side range check): kf_kv_append with
    device starts and kf_attn_append_decode with device lengths take a
    host-side bound on those positions and reject, before any launch, a call
    whose range would leave the capacity (kv_append_cuda.cu:72-73); the caches
    stay unchanged. A device position beyond the bound it was given breaks the
    caller's promise: its rows are skipped, never written out of range."""
    from kotflash_amd import _hip

    b, hkv, hq, cap, d, n = 2, 2, 8, 256, 64, 4
    kc = torch.full((b, hkv, cap, d), float("nan"), device="cuda", dtype=F16)
    vc = torch.full_like(kc, float("nan"))
    kc[:, :, :200] = 0
    vc[:, :, :200] = 0
    k0, v0 = kc.clone(), vc.clone()
    nk = seeded((b, hkv, n, d), 341, dtype=F16)
    nv = seeded((b, hkv, n, d), 342, dtype=F16)
    q = seeded((b, hq, 1, d), 343, dtype=F16)
    starts = torch.tensor([100, 253], device="cuda")
    with pytest.raises(RuntimeError, match="exceeds cache capacity"):
        _hip.kv_append(kc, vc, nk, nv, start_dev=starts, max_start=253)
    lengths = torch.tensor([100, 253], device="cuda", dtype=torch.int32)
    out = torch.empty_like(q)
    splits = _hip.decode_num_splits(b, hq, hkv, 1, 253, d)
    ws = torch.empty(_hip.decode_workspace_bytes(b, hq, hkv, 1, d, splits + 1), device="cuda",
                     dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="exceeds cache capacity"):
        _hip.append_decode(q, kc, vc, nk, nv, out, None, lengths, past_length=0, max_length=253,
                           scale=0.125, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), k0.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), v0.view(torch.int16))
    # A bound that fits, with one device start (150) above it (120): that
    # sequence is skipped, the other written.
    starts = torch.tensor([100, 150], device="cuda")
    _hip.kv_append(kc, vc, nk, nv, start_dev=starts, max_start=120)
    torch.cuda.synchronize()
    assert torch.equal(kc[0, :, 100:104], nk[0]) and torch.equal(vc[0, :, 100:104], nv[0])
    assert torch.equal(kc[1].view(torch.int16), k0[1].view(torch.int16))
    assert torch.equal(vc[1].view(torch.int16), v0[1].view(torch.int16))


def test_expanded_start_and_strided_seqlens_are_read_as_values():
    """Index tensors that are views (a stride-0 expand, a strided slice) are
    read by value, not as raw memory."""
    from kotflash_amd.kernels.hip_decode import attention_decode_ragged

    kc = torch.zeros((4, 2, 40, 64), device="cuda", dtype=F16)
    vc = torch.zeros_like(kc)
    nk = seeded((4, 2, 3, 64), 331, dtype=F16)
    nv = seeded((4, 2, 3, 64), 332, dtype=F16)
    start = torch.full((1,), 7, device="cuda", dtype=torch.int64).expand(4)
    assert start.stride() == (0,)
    append_kv_hip(kc, vc, nk, nv, start)
    assert torch.equal(kc[:, :, 7:10], nk) and torch.equal(vc[:, :, 7:10], nv)
    assert (kc[:, :, :7] == 0).all() and (kc[:, :, 10:] == 0).all()

    b, hkv, hq, cap, d = 3, 2, 8, 2048, 64
    kc = seeded((b, hkv, cap, d), 333, dtype=F16)
    vc = seeded((b, hkv, cap, d), 334, dtype=F16)
    q = seeded((b, hq, 2, d), 335, dtype=F16)
    lengths = [1500, 2048, 1100]
    wide = torch.tensor([[x, -5] for x in lengths], device="cuda", dtype=torch.int32)
    seqlens = wide[:, 0]
    assert seqlens.stride() == (2,)
    out = attention_decode_ragged(q, kc, vc, seqlens, max_seqlen=max(lengths), scale=0.125,
                                  host_lengths=lengths)
    for i, n in enumerate(lengths):
        eo, _ = reference_fp32(q[i:i + 1], kc[i:i + 1, :, :n], vc[i:i + 1, :, :n], causal=False,
                               scale=0.125)
        assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"seq {i}")
