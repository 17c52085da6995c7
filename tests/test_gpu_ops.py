"""The torch.library ops on the GPU: parity with the fp32 reference through
the ops, their use from torch.compile (dynamo + AOTAutograd tracing the fake
implementations and the registered backward, no graph break), and the
mutating cache append."""
import math

import pytest
import torch

import kotflash_amd as kf
import kotflash_amd.ops  # noqa: F401
from tests.gpu_helpers import BWD_TOL, FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_attn_ops_forward_backward(dtype):
    q = seeded((2, 8, 150, 64), 71, dtype=dtype).requires_grad_(True)
    k = seeded((2, 2, 170, 64), 72, dtype=dtype).requires_grad_(True)
    v = seeded((2, 2, 170, 64), 73, dtype=dtype).requires_grad_(True)
    do = seeded((2, 8, 150, 64), 74, dtype=dtype)
    out, lse = torch.ops.kotflash_amd.attn_fwd(q, k, v, True, 0.125)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), do)
    eo, el, (eq, ek, ev) = reference_fp32(q, k, v, causal=True, scale=0.125, with_grad_out=do)
    assert_close(out, eo, **FWD_TOL[dtype], what="O")
    assert_close(lse, el, **FWD_TOL[dtype], what="LSE")
    for g, e, n in ((dq, eq, "dQ"), (dk, ek, "dK"), (dv, ev, "dV")):
        assert_close(g, e, **BWD_TOL[dtype], what=n)


def test_torch_compile_traces_the_ops_without_graph_breaks():
    """fullgraph=True fails on any graph break; aot_eager runs the traced
    forward and backward graphs eagerly (no code generation needed)."""
    q = seeded((1, 4, 128, 64), 81, dtype=F16).requires_grad_(True)
    k = seeded((1, 2, 128, 64), 82, dtype=F16).requires_grad_(True)
    v = seeded((1, 2, 128, 64), 83, dtype=F16).requires_grad_(True)

    def loss_fn(q, k, v):
        out = torch.ops.kotflash_amd.attn_fwd(q, k, v, True, 1 / math.sqrt(64))[0]
        return (out.float() * out.float()).sum()

    compiled = torch.compile(loss_fn, backend="aot_eager", fullgraph=True)
    lc = compiled(q, k, v)
    gc = torch.autograd.grad(lc, (q, k, v))
    le = loss_fn(q, k, v)
    ge = torch.autograd.grad(le, (q, k, v))
    assert torch.equal(lc, le)
    for a, b in zip(gc, ge):
        assert torch.equal(a, b)


def test_public_attention_under_torch_compile():
    q = seeded((2, 4, 96, 128), 91, dtype=BF16).requires_grad_(True)
    k = seeded((2, 4, 96, 128), 92, dtype=BF16).requires_grad_(True)
    v = seeded((2, 4, 96, 128), 93, dtype=BF16).requires_grad_(True)
    do = seeded((2, 4, 96, 128), 94, dtype=BF16)
    fn = torch.compile(lambda q, k, v: kf.attention(q, k, v, causal=False, backend="hip"),
                       backend="aot_eager")
    out = fn(q, k, v)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), do)
    eo, _, (eq, ek, ev) = reference_fp32(q, k, v, causal=False, with_grad_out=do)
    assert_close(out, eo, **FWD_TOL[BF16], what="compiled O")
    for g, e, n in ((dq, eq, "dQ"), (dk, ek, "dK"), (dv, ev, "dV")):
        assert_close(g, e, **BWD_TOL[BF16], what=f"compiled {n}")


def test_decode_op_matches_reference():
    q = seeded((2, 8, 1, 64), 101, dtype=F16)
    k = seeded((2, 2, 3000, 64), 102, dtype=F16)
    v = seeded((2, 2, 3000, 64), 103, dtype=F16)
    out = torch.ops.kotflash_amd.decode(q, k, v, 0.125)
    eo, _ = reference_fp32(q, k, v, causal=False, scale=0.125)
    assert_close(out, eo, **FWD_TOL[F16], what="decode O")


def test_kv_append_op_writes_only_the_slots():
    kc = torch.full((2, 2, 64, 64), float("nan"), dtype=F16, device="cuda")
    vc = kc.clone()
    nk = seeded((2, 2, 5, 64), 111, dtype=F16)
    nv = seeded((2, 2, 5, 64), 112, dtype=F16)
    torch.ops.kotflash_amd.kv_append_(kc, vc, nk, nv, 30)
    assert torch.equal(kc[:, :, 30:35], nk) and torch.equal(vc[:, :, 30:35], nv)
    assert torch.isnan(kc[:, :, :30]).all() and torch.isnan(kc[:, :, 35:]).all()
    assert torch.isnan(vc[:, :, :30]).all() and torch.isnan(vc[:, :, 35:]).all()
    with pytest.raises(ValueError, match="capacity"):
        torch.ops.kotflash_amd.kv_append_(kc, vc, nk, nv, 60)


def test_append_decode_op_writes_the_slot_and_attends():
    kc = torch.full((2, 2, 2048, 64), float("nan"), dtype=F16, device="cuda")
    vc = kc.clone()
    kc[:, :, :1500] = seeded((2, 2, 1500, 64), 121, dtype=F16)
    vc[:, :, :1500] = seeded((2, 2, 1500, 64), 122, dtype=F16)
    nk = seeded((2, 2, 1, 64), 123, dtype=F16)
    nv = seeded((2, 2, 1, 64), 124, dtype=F16)
    q = seeded((2, 8, 1, 64), 125, dtype=F16)
    out = torch.ops.kotflash_amd.append_decode_(q, kc, vc, nk, nv, 1500, 0.125)
    assert torch.equal(kc[:, :, 1500:1501], nk) and torch.equal(vc[:, :, 1500:1501], nv)
    assert torch.isnan(kc[:, :, 1501:]).all() and torch.isnan(vc[:, :, 1501:]).all()
    eo, _ = reference_fp32(q, kc[:, :, :1501], vc[:, :, :1501], causal=False, scale=0.125)
    assert_close(out, eo, **FWD_TOL[F16], what="append_decode_ O")
