"""BASELINE config 5 in full: all 64 steps, all 8 sequences, both append +
decode paths, against dense fp32 attention.

Same inputs as bench.py's config 5 loop (seed 500): cache [8, 8, 32768, 64]
fp16 prefilled to per-sequence lengths U[4096, 28000] with NaN in every
unused slot; step t draws n in [1, 16], appends new K/V (seeds 600 + t,
700 + t) at each sequence's own position and decodes q [8, 32, n, 64]
(seed 800 + t) non-causally over each sequence's first L_b + n keys. The
append must be bit-exact every step (reference kv_append_cuda.cu:12-40) with
the NaN sentinels after it untouched; O of every sequence must match fp32
attention on its visible prefix within the fp16 tolerance.
"""
import pytest
import torch

from kotflash_amd.cache import RaggedKVCache
from tests.gpu_helpers import FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16 = torch.float16
B, HKV, CAP, D, HQ, STEPS, SEED = 8, 8, 32768, 64, 32, 64, 500


def _prefilled_cache():
    g = torch.Generator().manual_seed(SEED)
    lengths = torch.randint(4096, 28001, (B,), generator=g).tolist()
    ns = [int(torch.randint(1, 17, (1,), generator=g)) for _ in range(STEPS)]
    cache = RaggedKVCache(B, HKV, CAP, D, device="cuda", dtype=F16)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    for i, n in enumerate(lengths):
        cache.k[i, :, :n] = seeded((HKV, n, D), 510 + i, dtype=F16)
        cache.v[i, :, :n] = seeded((HKV, n, D), 520 + i, dtype=F16)
    cache.set_lengths(lengths)
    return cache, ns


@pytest.mark.parametrize("path", ["two_launch", "fused"])
def test_config5_all_steps_all_sequences(path):
    cache, ns = _prefilled_cache()
    print(f"config 5 full, path={path}, n per step={ns}", flush=True)
    worst = 0.0
    for t, n in enumerate(ns):
        nk = seeded((B, HKV, n, D), 600 + t, dtype=F16)
        nv = seeded((B, HKV, n, D), 700 + t, dtype=F16)
        q = seeded((B, HQ, n, D), 800 + t, dtype=F16)
        before = list(cache.lengths)
        with torch.inference_mode():
            if path == "fused":
                out = cache.append_and_attend(q, nk, nv, append_backend="fused",
                                              attention_backend="hip")
            else:
                cache.append(nk, nv, backend="hip")
                out = cache.attend(q, backend="hip")
        assert cache.lengths == [x + n for x in before]
        for i, s in enumerate(before):
            assert torch.equal(cache.k[i, :, s:s + n], nk[i]), f"step {t} seq {i} K append"
            assert torch.equal(cache.v[i, :, s:s + n], nv[i]), f"step {t} seq {i} V append"
            assert torch.isnan(cache.k[i, :, s + n]).all() and torch.isnan(cache.v[i, :, s + n]).all()
        for i in range(B):
            kv, vv = cache.view(i)
            eo, _ = reference_fp32(q[i:i + 1], kv, vv, causal=False)
            assert_close(out[i:i + 1], eo, **FWD_TOL[F16], what=f"{path} step {t} seq {i}")
            worst = max(worst, float((out[i:i + 1].float() - eo).abs().max()))
    # Every slot past the final lengths still holds its NaN sentinel.
    for i, s in enumerate(cache.lengths):
        assert torch.isnan(cache.k[i, :, s:]).all() and torch.isnan(cache.v[i, :, s:]).all()
    print(f"config 5 full, path={path}: 64 steps x 8 sequences, max |O - fp32| = {worst:.2e}",
          flush=True)
