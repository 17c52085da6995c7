"""CPU behaviour of the public API (the reference's tests/test_api.py and
tests/test_attention.py contract, re-expressed against kotflash_amd)."""
import math

import pytest
import torch
import torch.nn.functional as F

import kotflash_amd
from kotflash_amd import attention
from kotflash_amd.attention import _blockwise_backward, _sdpa, _sdpa_expanded


def test_package_exports():
    assert set(kotflash_amd.__all__) >= {"attention", "triton_available", "triton_turing_supported"}
    assert kotflash_amd.triton_available() is False
    assert kotflash_amd.triton_turing_supported() is False
    assert kotflash_amd.hip_available() is False  # no GPU here


def test_t4_gate_needs_every_condition(monkeypatch):
    """The reference's exact-stack T4 gate (kotflash/attention.py:74-87):
    true only for Triton on SM75 with CUDA 12.4, a Tesla T4 and torch 2.6.0,
    and false when any one of them differs (it is false on ROCm)."""
    import importlib

    impl = importlib.import_module("kotflash_amd.attention")  # the module, not the function
    gate = impl._is_measured_t4_runtime.__wrapped__  # past its per-device cache
    assert gate(0) is False
    stack = {
        "triton": ("triton_turing_supported", lambda: True),
        "cuda": ("version.cuda", "12.4"),
        "available": ("cuda.is_available", lambda: True),
        "capability": ("cuda.get_device_capability", lambda d: (7, 5)),
        "name": ("cuda.get_device_name", lambda d: "Tesla T4"),
        "torch": ("__version__", "2.6.0+cu124"),
    }
    wrong = {"triton": lambda: False, "cuda": None, "available": lambda: False,
             "capability": lambda d: (8, 0), "name": lambda d: "NVIDIA A10", "torch": "2.5.1"}

    def apply(mp, key, value):
        where, val = stack[key]
        if where == "triton_turing_supported":
            mp.setattr(impl, "triton_turing_supported", value)
        elif where.startswith("cuda."):
            mp.setattr(torch.cuda, where.split(".", 1)[1], value)
        elif where == "version.cuda":
            mp.setattr(torch.version, "cuda", value)
        else:
            mp.setattr(torch, "__version__", value)

    with monkeypatch.context() as mp:
        for key, (_, val) in stack.items():
            apply(mp, key, val)
        assert gate(0) is True
    for off in stack:
        with monkeypatch.context() as mp:
            for key, (_, val) in stack.items():
                apply(mp, key, wrong[key] if key == off else val)
            assert not gate(0), off


def test_sdpa_matches_torch_mha():
    torch.manual_seed(0)
    q = torch.randn(2, 4, 17, 32)
    k = torch.randn(2, 4, 19, 32)
    v = torch.randn_like(k)
    torch.testing.assert_close(attention(q, k, v, backend="sdpa"), F.scaled_dot_product_attention(q, k, v))


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_gqa_unequal_lengths(causal):
    torch.manual_seed(1)
    q = torch.randn(2, 8, 6, 32)
    k = torch.randn(2, 2, 9, 32)
    v = torch.randn_like(k)
    expected = F.scaled_dot_product_attention(
        q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), is_causal=causal)
    torch.testing.assert_close(attention(q, k, v, causal=causal, backend="sdpa"), expected)


def test_auto_on_cpu_is_sdpa():
    torch.manual_seed(2)
    q = torch.randn(1, 8, 11, 16)
    k = torch.randn(1, 2, 13, 16)
    v = torch.randn_like(k)
    torch.testing.assert_close(attention(q, k, v), attention(q, k, v, backend="sdpa"))


@pytest.mark.parametrize("expanded", [False, True])
def test_default_scale_is_not_forwarded(monkeypatch, expanded):
    q = torch.randn(1, 4, 5, 16)
    k = torch.randn(1, 1, 7, 16)
    v = torch.randn_like(k)
    seen = {}

    def fake_sdpa(query, key, value, **kwargs):
        seen["kwargs"] = kwargs
        seen["heads"] = key.shape[1]
        return torch.zeros_like(query)

    monkeypatch.setattr(F, "scaled_dot_product_attention", fake_sdpa)
    (_sdpa_expanded if expanded else _sdpa)(q, k, v, causal=False, scale=1.0 / math.sqrt(16))
    assert "scale" not in seen["kwargs"]
    assert seen["heads"] == (4 if expanded else 1)
    (_sdpa_expanded if expanded else _sdpa)(q, k, v, causal=False, scale=0.2)
    assert seen["kwargs"]["scale"] == 0.2


def test_custom_scale_matches_scaled_query():
    torch.manual_seed(2)
    q = torch.randn(1, 2, 5, 16)
    k = torch.randn(1, 2, 7, 16)
    v = torch.randn_like(k)
    expected = F.scaled_dot_product_attention(q * (0.125 * math.sqrt(16)), k, v)
    torch.testing.assert_close(attention(q, k, v, scale=0.125, backend="sdpa"), expected)


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_rejects_nonfinite_scale(bad):
    q = torch.randn(1, 1, 2, 16)
    with pytest.raises(ValueError, match="finite"):
        attention(q, q, q, scale=bad, backend="sdpa")


def test_rejects_non_numeric_scale_and_bad_causal_and_backend():
    q = torch.randn(1, 1, 2, 16)
    with pytest.raises(TypeError, match="scale"):
        attention(q, q, q, scale="x")
    with pytest.raises(TypeError, match="causal"):
        attention(q, q, q, causal=1)
    with pytest.raises(ValueError, match="backend"):
        attention(q, q, q, backend="cuda")


@pytest.mark.parametrize(
    "shapes,match",
    [
        (((2, 3, 5, 8), (2, 2, 7, 8), (2, 2, 7, 8)), "divisible"),
        (((2, 4, 5, 8), (1, 2, 7, 8), (1, 2, 7, 8)), "Batch dimensions"),
        (((2, 4, 5, 8), (2, 2, 7, 8), (2, 2, 6, 8)), "K and V shapes"),
        (((2, 4, 5, 8), (2, 2, 7, 16), (2, 2, 7, 16)), "head dimensions"),
        (((2, 4, 0, 8), (2, 2, 7, 8), (2, 2, 7, 8)), "Sequence"),
        (((0, 4, 5, 8), (0, 2, 7, 8), (0, 2, 7, 8)), "Batch dimension must be non-zero"),
        (((2, 4, 5, 0), (2, 2, 7, 0), (2, 2, 7, 0)), "Head dimension must be non-zero"),
        (((2, 4, 5), (2, 2, 7, 8), (2, 2, 7, 8)), "layout"),
    ],
)
def test_validation_errors(shapes, match):
    q, k, v = (torch.randn(*s) for s in shapes)
    with pytest.raises(ValueError, match=match):
        attention(q, k, v)


def test_dtype_mismatch_and_type_errors():
    q = torch.randn(1, 2, 3, 8)
    with pytest.raises(ValueError, match="dtypes"):
        attention(q, q.double(), q)
    with pytest.raises(TypeError, match="torch.Tensor"):
        attention(q, q.numpy(), q)


def test_explicit_hip_backend_fails_loudly_on_cpu():
    q = torch.randn(1, 2, 16, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="gfx950"):
        attention(q, q, q, backend="hip")
    with pytest.raises(RuntimeError, match="gfx950"):
        attention(q, q, q, backend="triton")


def _autograd_grads(q, k, v, causal, scale):
    qr, kr, vr = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    g = q.shape[1] // k.shape[1]
    ke, ve = kr.repeat_interleave(g, 1), vr.repeat_interleave(g, 1)
    s = torch.matmul(qr, ke.transpose(-2, -1)) * scale
    if causal:
        mask = torch.arange(k.shape[2])[None, :] > torch.arange(q.shape[2])[:, None]
        s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, -1)
    out = torch.softmax(s, -1) @ ve
    do = torch.randn_like(out)
    grads = torch.autograd.grad(out, (qr, kr, vr), do)
    return out.detach(), lse.detach(), do, grads


@pytest.mark.parametrize(
    "hq,hkv,sq,sk,causal",
    [(2, 2, 5, 7, False), (4, 2, 5, 7, False), (2, 2, 5, 7, True),
     (2, 1, 7, 5, True), (4, 2, 5, 9, False), (2, 2, 9, 5, True)],
)
def test_blockwise_backward_matches_autograd(hq, hkv, sq, sk, causal):
    torch.manual_seed(19)
    q = torch.randn(2, hq, sq, 16)
    k = torch.randn(2, hkv, sk, 16)
    v = torch.randn(2, hkv, sk, 16)
    scale = 1 / math.sqrt(16)
    out, lse, do, expected = _autograd_grads(q, k, v, causal, scale)
    got = _blockwise_backward(q, k, v, out, lse, do, causal=causal, scale=scale,
                              q_block=3, kv_block=2)
    for a, b in zip(got, expected):
        torch.testing.assert_close(a, b, rtol=3e-4, atol=3e-5)
