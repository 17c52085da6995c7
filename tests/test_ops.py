"""The torch.library registration of the HIP kernels (no GPU needed): the
ops exist with the expected schemas, their fake implementations give the
output shapes, and autograd runs attn_fwd's registered backward."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import kotflash_amd.ops  # noqa: F401  (registers the ops)


def test_ops_registered_with_schemas():
    ns = torch.ops.kotflash_amd
    fwd = str(ns.attn_fwd.default._schema)
    bwd = str(ns.attn_bwd.default._schema)
    app = str(ns.kv_append_.default._schema)
    dec = str(ns.decode.default._schema)
    assert "bool causal, float scale) -> (Tensor, Tensor)" in fwd
    assert "Tensor grad_out, bool causal, float scale) -> (Tensor, Tensor, Tensor)" in bwd
    assert "float scale) -> Tensor" in dec
    # Both caches are declared as mutated; the new values are not.
    assert "Tensor(a0!) k_cache" in app and "Tensor(a1!) v_cache" in app
    assert "Tensor new_k" in app and "Tensor new_v" in app and "-> ()" in app


@pytest.mark.parametrize("shape", [
    # (B, Hq, Hkv, Sq, Sk, D)
    (2, 8, 2, 100, 120, 64),   # GQA
    (1, 4, 4, 33, 33, 128),    # MHA
    (3, 6, 1, 5, 700, 72),     # MQA, unpadded head_dim
])
def test_fake_forward_and_registered_backward(shape):
    b, hq, hkv, sq, sk, d = shape
    with FakeTensorMode():
        q = torch.empty(b, hq, sq, d, dtype=torch.float16, requires_grad=True)
        k = torch.empty(b, hkv, sk, d, dtype=torch.float16, requires_grad=True)
        v = torch.empty(b, hkv, sk, d, dtype=torch.float16, requires_grad=True)
        out, lse = torch.ops.kotflash_amd.attn_fwd(q, k, v, True, 0.125)
        assert out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous()
        assert lse.shape == (b, hq, sq) and lse.dtype == torch.float32
        assert out.requires_grad and not lse.requires_grad
        dq, dk, dv = torch.autograd.grad(out, (q, k, v), torch.empty_like(out))
        assert (dq.shape, dk.shape, dv.shape) == (q.shape, k.shape, v.shape)
        assert dk.dtype == k.dtype


def test_fake_decode_shape():
    with FakeTensorMode():
        q = torch.empty(2, 8, 1, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 2, 4096, 64, dtype=torch.bfloat16)
        assert torch.ops.kotflash_amd.decode(q, k, k, 0.125).shape == q.shape


def test_kv_append_rejects_host_tensors():
    cache = torch.zeros(1, 2, 16, 64, dtype=torch.float16)
    new = torch.ones(1, 2, 1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="requires GPU tensors"):
        torch.ops.kotflash_amd.kv_append_(cache, cache.clone(), new, new, 3)
    assert not cache.any()


def test_append_decode_op_schema_and_fake():
    sch = str(torch.ops.kotflash_amd.append_decode_.default._schema)
    assert "Tensor(a1!) k_cache" in sch and "Tensor(a2!) v_cache" in sch
    assert "Int past_length, float scale) -> Tensor" in sch
    with FakeTensorMode():
        q = torch.empty(2, 8, 1, 64, dtype=torch.float16)
        kc = torch.empty(2, 2, 4096, 64, dtype=torch.float16)
        new = torch.empty(2, 2, 1, 64, dtype=torch.float16)
        out = torch.ops.kotflash_amd.append_decode_(q, kc, kc.clone(), new, new, 100, 0.125)
        assert out.shape == q.shape and out.dtype == q.dtype
