"""The reference's own import lines resolve against this build (CPU only).

Each import statement below is spelled exactly as in a reference file
(cited), so a caller of the reference keeps its code unchanged. The names
must be the objects that implement them, not stand-ins.
"""
import importlib


def test_reference_test_and_example_imports():
    # reference tests/test_attention.py:8-9
    from kotflash import attention
    from kotflash.attention import _blockwise_backward, _sdpa, _sdpa_expanded
    # reference tests/test_kv_cache.py:7
    from kotflash.cache import append_kv_cache, decode_step
    # reference tests/test_planning.py:5-7
    from kotflash._planning import (
        INT32_MAX, check_int32_indexing, split_kv_plan, t4_profile_for_shapes,
    )
    # reference tests/test_preallocated_cache.py:6 and tests/test_cuda_append.py:8
    from kotflash.cache import PreallocatedKVCache
    # reference tests/test_triton.py:7-8 and examples/gqa_kv_cache_decode.py:13-14
    from kotflash import attention as attention2, triton_turing_supported
    from kotflash.attention import _t4_profile_backend
    # reference benchmarks/benchmark_decode.py:26-27
    from kotflash.cache import append_kv_cache as append2, PreallocatedKVCache as Cache2

    import kotflash_amd
    impl = importlib.import_module("kotflash_amd.attention")
    assert attention is attention2 is kotflash_amd.attention
    assert _blockwise_backward is impl._blockwise_backward
    assert _sdpa is impl._sdpa and _sdpa_expanded is impl._sdpa_expanded
    assert _t4_profile_backend is impl._t4_profile_backend
    cache = importlib.import_module("kotflash_amd.cache")
    assert PreallocatedKVCache is Cache2 is cache.PreallocatedKVCache
    assert append_kv_cache is append2 is cache.append_kv_cache
    assert decode_step is cache.decode_step
    assert INT32_MAX == 2**31 - 1 and callable(check_int32_indexing)
    assert split_kv_plan(1, 2048, 64, causal=False).num_splits == 16
    assert t4_profile_for_shapes((2, 8, 1024, 64), (2, 2, 1024, 64), (2, 2, 1024, 64),
                                 causal=True, scale=0.125, contiguous=True) == "triton"
    assert triton_turing_supported() is False


def test_package_and_kernel_module_names():
    import kotflash
    import kotflash.kernels.triton_backward as tb
    from kotflash.kernels.triton_decode import (
        attention_forward_strided_append, attention_forward_strided_decode,
        strided_decode_supported,
    )
    from kotflash.kernels.triton_forward import (
        attention_forward, triton_available, triton_turing_supported,
    )
    from kotflash._cuda_append import append_kv_cuda

    hip_decode = importlib.import_module("kotflash_amd.kernels.hip_decode")
    assert strided_decode_supported is hip_decode.strided_decode_supported
    assert attention_forward_strided_decode is hip_decode.attention_forward_strided_decode
    assert attention_forward_strided_append is hip_decode.attention_forward_strided_append
    assert tb.attention_backward is importlib.import_module(
        "kotflash_amd.kernels.hip_backward").attention_backward
    assert attention_forward is importlib.import_module(
        "kotflash_amd.kernels.hip_forward").attention_forward
    assert triton_available() is False and triton_turing_supported() is False
    assert append_kv_cuda is importlib.import_module("kotflash_amd._hip_append").append_kv_hip
    # As in the reference, the package attribute is the function and the
    # submodule is reachable through sys.modules.
    assert callable(kotflash.attention) and kotflash.__all__[0] == "attention"
    assert importlib.import_module("kotflash.attention").__name__ == "kotflash_amd.attention"
    assert kotflash.cache is importlib.import_module("kotflash_amd.cache")


def test_monkeypatching_through_the_reference_name_reaches_the_implementation(monkeypatch):
    """Patching ``kotflash.attention._sdpa`` (a module attribute under the
    reference's name) changes what ``attention(backend="sdpa")`` runs."""
    import torch

    import kotflash
    calls = []
    mod = importlib.import_module("kotflash.attention")
    real = mod._sdpa

    def spy(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    monkeypatch.setattr(mod, "_sdpa", spy)
    q = torch.randn(1, 2, 4, 8)
    kotflash.attention(q, q, q, backend="sdpa")
    assert calls == [1]


def test_launchers_accept_the_reference_tuning_keywords():
    """attention_forward / attention_backward take the reference launchers'
    tuning keywords (triton_forward.py:372-376, triton_backward.py:335-339),
    as its tile tuner passes them (benchmarks/tune_triton_tiles.py:186-190);
    bad values get the reference's messages (triton_forward.py:392-395). On
    CPU tensors the call then stops at the device check, after the keywords
    were accepted."""
    import inspect

    import pytest
    import torch
    from kotflash.kernels.triton_backward import attention_backward
    from kotflash.kernels.triton_forward import attention_forward

    fwd = inspect.signature(attention_forward).parameters
    bwd = inspect.signature(attention_backward).parameters
    for params, defaults in ((fwd, (64, 32, 4, 2)), (bwd, (32, 64, 4, 1))):
        for name, default in zip(("block_m", "block_n", "num_warps", "num_stages"), defaults):
            assert params[name].kind is inspect.Parameter.KEYWORD_ONLY
            assert params[name].default == default
    q = torch.zeros(1, 2, 16, 64, dtype=torch.float16)
    k = torch.zeros(1, 1, 16, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="block_m and block_n must be positive"):
        attention_forward(q, k, k, causal=True, scale=0.125, block_m=0)
    with pytest.raises(ValueError, match="num_warps and num_stages must be positive"):
        attention_forward(q, k, k, causal=True, scale=0.125, num_stages=0)
    with pytest.raises(ValueError, match="block_m and block_n must be positive"):
        attention_backward(q, k, k, q, q[..., 0].float(), q, causal=True, scale=0.125, block_n=-1)
    with pytest.raises((RuntimeError, ValueError), match="GPU|gfx950|HIP|device|CUDA"):
        attention_forward(q, k, k, causal=True, scale=0.125, block_m=32, block_n=64,
                          num_warps=8, num_stages=1)
    with pytest.raises((RuntimeError, ValueError), match="GPU|gfx950|HIP|device|CUDA"):
        attention_backward(q, k, k, q, q[..., 0].float(), q, causal=True, scale=0.125,
                           block_m=64, block_n=128, num_warps=8, num_stages=2)
