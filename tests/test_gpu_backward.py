"""Backward parity on the GPU: HIP dQ/dK/dV (through the C ABI) vs the
golden fixtures, the oracle and fp32 autograd, including GQA group sums,
head-dim tails and the BASELINE configurations."""
import math

import numpy as np
import pytest
import torch

from kotflash_amd import attention
from kotflash_amd.kernels.hip_backward import attention_backward
from kotflash_amd.kernels.hip_forward import attention_forward
from oracle import attention_oracle as orc
from tests.conftest import GOLDEN_ATTN_CASES
from tests.gpu_helpers import (BWD_TOL, BWD_TOL_BF16_SHORT, FWD_TOL, assert_close, error_stats,
                                reference_fp32, seeded)

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


def _check_grads(q, k, v, do, causal, dtype, what, bwd_tol=None):
    out, lse = attention_forward(q, k, v, causal=causal, scale=1 / math.sqrt(q.shape[-1]))
    dq, dk, dv = attention_backward(q, k, v, out, lse, do, causal=causal,
                                    scale=1 / math.sqrt(q.shape[-1]))
    eo, el, (eq, ek, ev) = reference_fp32(q, k, v, causal=causal, with_grad_out=do)
    assert dq.dtype == q.dtype and dk.shape == k.shape and dv.shape == v.shape
    tol = BWD_TOL[dtype] if bwd_tol is None else bwd_tol
    assert_close(out, eo, **FWD_TOL[dtype], what=f"{what} O")
    assert_close(dq, eq, **tol, what=f"{what} dQ")
    assert_close(dk, ek, **tol, what=f"{what} dK")
    assert_close(dv, ev, **tol, what=f"{what} dV")


@pytest.mark.parametrize("name", GOLDEN_ATTN_CASES)
def test_backward_matches_golden(golden, name):
    b, hq, hkv, sq, sk, d, causal = (int(x) for x in golden[f"{name}/meta"])
    q, k, v, do = (torch.from_numpy(golden[f"{name}/{x}"]).cuda() for x in ("q", "k", "v", "do"))
    out, lse = attention_forward(q, k, v, causal=bool(causal), scale=1 / math.sqrt(d))
    dq, dk, dv = attention_backward(q, k, v, out, lse, do, causal=bool(causal), scale=1 / math.sqrt(d))
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert_close(got, torch.from_numpy(golden[f"{name}/{key}"]), **BWD_TOL[F16],
                     what=f"{name} {key}")


def test_backward_matches_oracle_with_stored_o():
    """The oracle restates the kernels' numerics: delta from the stored fp16 O
    and the kernel's own LSE, P and dS rounded to fp16 before their products."""
    q = seeded((1, 4, 150, 64), 71, dtype=F16)
    k = seeded((1, 2, 170, 64), 72, dtype=F16)
    v = seeded((1, 2, 170, 64), 73, dtype=F16)
    do = seeded((1, 4, 150, 64), 74, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=True, scale=0.125)
    dq, dk, dv = attention_backward(q, k, v, out, lse, do, causal=True, scale=0.125)
    n = lambda t: t.detach().cpu().float().numpy().astype(np.float64)
    eq, ek, ev = orc.backward_blockwise(n(q), n(k), n(v), n(out), n(lse), n(do), causal=True,
                                        scale=0.125, p_dtype=np.float16)
    for got, exp, key in ((dq, eq, "dq"), (dk, ek, "dk"), (dv, ev, "dv")):
        assert_close(got, torch.from_numpy(exp), atol=4e-3, rtol=4e-3, what=key)


@pytest.mark.parametrize("hq,hkv,sq,sk,d,causal", [
    # The reference's backward cases (tests/test_triton.py:160-174).
    (4, 4, 64, 80, 32, False),
    (8, 2, 64, 80, 64, True),
    (8, 1, 80, 64, 32, True),
    (8, 2, 48, 64, 72, False),
    (4, 4, 48, 64, 96, True),
    (8, 1, 64, 48, 128, False),
    (8, 2, 1024, 1024, 64, True),
    (4, 1, 1024, 768, 32, False),
    (4, 2, 2048, 2048, 32, True),
    (8, 2, 1, 1024, 64, False),
])
@pytest.mark.parametrize("dtype", [F16, BF16])
def test_backward_reference_cases(hq, hkv, sq, sk, d, causal, dtype):
    q = seeded((1, hq, sq, d), 12, dtype=dtype)
    k = seeded((1, hkv, sk, d), 13, dtype=dtype)
    v = seeded((1, hkv, sk, d), 14, dtype=dtype)
    do = seeded((1, hq, sq, d), 15, dtype=dtype)
    short_bf16 = dtype == BF16 and max(sq, sk) <= 80
    _check_grads(q, k, v, do, causal, dtype, f"{(hq, hkv, sq, sk, d, causal)}",
                 bwd_tol=BWD_TOL_BF16_SHORT if short_bf16 else None)


@pytest.mark.parametrize("shape", [
    (3, 6, 3, 1000, 1000, 64, True),   # 9 KV groups: stream-K shares cross group boundaries
    (3, 6, 3, 1000, 1000, 64, False),
    (1, 2, 1, 500, 130, 64, True),   # Sq > Sk causal: keys seen by many rows
    (1, 2, 2, 70, 900, 128, True),   # keys beyond Sq never seen: zero dK/dV
    (2, 3, 1, 129, 131, 40, False),  # head_dim 40, ragged tiles
    (1, 2, 1, 33, 47, 20, True),     # padded head_dim
])
def test_backward_edge_shapes(shape):
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 81, dtype=F16)
    k = seeded((b, hkv, sk, d), 82, dtype=F16)
    v = seeded((b, hkv, sk, d), 83, dtype=F16)
    do = seeded((b, hq, sq, d), 84, dtype=F16)
    _check_grads(q, k, v, do, causal, F16, f"{shape}")


@pytest.mark.parametrize("shape", [
    (2, 8, 2, 1100, 1100, 128, True),  # tiled dQ, stream-K dK/dV with shared tiles
    (1, 6, 6, 700, 700, 96, False),    # 96-wide tile, non-causal MHA
    (1, 4, 2, 200, 300, 64, False),    # split dQ form (short problem), Sk > Sq
])
def test_backward_reads_strided_views_in_place(shape):
    """q/k/v and dO as [B, S, H, D] storage viewed as [B, H, S, D], the layout
    a model's projections produce: the kernels read them through their
    strides (no copy is made) and must match fp32 autograd."""
    from kotflash_amd.kernels._layout import prepare

    b, hq, hkv, sq, sk, d, causal = shape
    print(f"strided backward {shape}", flush=True)
    q = seeded((b, sq, hq, d), 85, dtype=F16).transpose(1, 2)
    k = seeded((b, sk, hkv, d), 86, dtype=F16).transpose(1, 2)
    v = seeded((b, sk, hkv, d), 87, dtype=F16).transpose(1, 2)
    do = seeded((b, sq, hq, d), 88, dtype=F16).transpose(1, 2)
    for t in (q, k, v, do):
        assert not t.is_contiguous() and prepare(t, d).data_ptr() == t.data_ptr()
    _check_grads(q, k, v, do, causal, F16, f"strided {shape}")


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_config3_forward_backward(dtype):
    """B=2, Hq=16, Hkv=4, S=4096, D=128, causal,
    q/k/v ~ 0.5 N(0,1), dO ~ N(0,1); dK/dV summed over the GQA group."""
    q = seeded((2, 16, 4096, 128), 301, dtype=dtype, scale=0.5)
    k = seeded((2, 4, 4096, 128), 302, dtype=dtype, scale=0.5)
    v = seeded((2, 4, 4096, 128), 303, dtype=dtype, scale=0.5)
    do = seeded((2, 16, 4096, 128), 304, dtype=dtype)
    _check_grads(q, k, v, do, True, dtype, "cfg3")


@pytest.mark.parametrize("head_dim", [72, 96])
def test_config4_forward_backward(head_dim):
    """B=4, H=12, S=2048, D in {72, 96}, non-causal MHA."""
    q = seeded((4, 12, 2048, head_dim), 401, dtype=F16)
    k = seeded((4, 12, 2048, head_dim), 402, dtype=F16)
    v = seeded((4, 12, 2048, head_dim), 403, dtype=F16)
    do = seeded((4, 12, 2048, head_dim), 404, dtype=F16)
    _check_grads(q, k, v, do, False, F16, f"cfg4 D={head_dim}")


def test_backward_is_deterministic():
    q = seeded((1, 8, 700, 64), 91, dtype=F16)
    k = seeded((1, 2, 700, 64), 92, dtype=F16)
    v = seeded((1, 2, 700, 64), 93, dtype=F16)
    do = seeded((1, 8, 700, 64), 94, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=True, scale=0.125)
    a = attention_backward(q, k, v, out, lse, do, causal=True, scale=0.125)
    b = attention_backward(q, k, v, out, lse, do, causal=True, scale=0.125)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_autograd_through_public_api(dtype):
    q = seeded((1, 4, 96, 64), 95, dtype=dtype).requires_grad_(True)
    k = seeded((1, 2, 96, 64), 96, dtype=dtype).requires_grad_(True)
    v = seeded((1, 2, 96, 64), 97, dtype=dtype).requires_grad_(True)
    do = seeded((1, 4, 96, 64), 98, dtype=dtype)
    out = attention(q, k, v, causal=True, backend="hip")
    grads = torch.autograd.grad(out, (q, k, v), do)
    _, _, exp = reference_fp32(q, k, v, causal=True, with_grad_out=do)
    for g, e, n in zip(grads, exp, "qkv"):
        assert_close(g, e, **BWD_TOL[dtype], what=f"d{n}")
    # Short query with grad goes through the split-KV forward + backward.
    qs = seeded((1, 4, 3, 64), 99, dtype=dtype).requires_grad_(True)
    ks = seeded((1, 2, 2048, 64), 100, dtype=dtype).requires_grad_(True)
    vs = seeded((1, 2, 2048, 64), 101, dtype=dtype).requires_grad_(True)
    dos = seeded((1, 4, 3, 64), 102, dtype=dtype)
    outs = attention(qs, ks, vs, causal=False, backend="hip")
    grads = torch.autograd.grad(outs, (qs, ks, vs), dos)
    _, _, exp = reference_fp32(qs, ks, vs, causal=False, with_grad_out=dos)
    for g, e, n in zip(grads, exp, "qkv"):
        assert_close(g, e, **BWD_TOL[dtype], what=f"split d{n}")


@pytest.mark.parametrize("shape", [
    # (B, Hq, Hkv, Sq, Sk, D, causal). The dK/dV schedule walks a KV group's
    # key tiles long and short alternately and places stream-K boundaries by
    # cost; these cases stress it.
    (1, 8, 1, 4096, 4096, 64, True),    # one KV group: long rows cut into many shares
    (1, 4, 2, 1100, 1100, 64, True),    # an odd number (9) of seen key tiles
    (2, 4, 2, 300, 1000, 64, True),     # 3 seen key tiles of 8, the rest never seen
    (1, 2, 1, 2500, 700, 128, True),    # Sq > Sk causal
    (2, 8, 2, 1024, 1024, 128, False),  # equal rows, shares on row boundaries
])
def test_backward_schedule_shapes(shape):
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 85, dtype=F16)
    k = seeded((b, hkv, sk, d), 86, dtype=F16)
    v = seeded((b, hkv, sk, d), 87, dtype=F16)
    do = seeded((b, hq, sq, d), 88, dtype=F16)
    _check_grads(q, k, v, do, causal, F16, f"{shape}")


@pytest.mark.parametrize("shape", [
    # (B, Hq, Hkv, Sq, Sk, D, causal): the split dQ form with one-stage rings
    # (D > 64) in bf16.
    (1, 2, 1, 2500, 700, 128, True),
    (2, 16, 4, 512, 512, 96, True),
])
def test_backward_split_dq_bf16(shape):
    """dQ (the split form under test) at the bf16 bar |a - b| <= 1e-2 +
    1e-2 |ref|. dK/dV come from the dK/dV kernel; at the second shape that bar
    is at the edge of bf16 itself: torch's bf16 SDPA backward on the same
    inputs misses it on 7 dK and 4 dV elements (up to 1.2x and 1.44x the
    bound), this build on one dK element (1.009x). They are held to the
    no-worse-than-torch criterion of test_bf16_gradients_no_worse_than_torch."""
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 89, dtype=BF16)
    k = seeded((b, hkv, sk, d), 90, dtype=BF16)
    v = seeded((b, hkv, sk, d), 91, dtype=BF16)
    do = seeded((b, hq, sq, d), 92, dtype=BF16)
    scale = 1 / math.sqrt(d)
    out, lse = attention_forward(q, k, v, causal=causal, scale=scale)
    dq, dk, dv = attention_backward(q, k, v, out, lse, do, causal=causal, scale=scale)
    _, _, (eq, ek, ev) = reference_fp32(q, k, v, causal=causal, with_grad_out=do)
    assert_close(dq, eq, **BWD_TOL[BF16], what=f"{shape} dQ")
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    g = hq // hkv
    to = torch.nn.functional.scaled_dot_product_attention(
        qq, kk.repeat_interleave(g, 1).contiguous(), vv.repeat_interleave(g, 1).contiguous(),
        is_causal=causal)
    _, tk, tv = torch.autograd.grad(to, (qq, kk, vv), do)
    for a, t, e, n in ((dk, tk, ek, "k"), (dv, tv, ev, "v")):
        ea = float((a.float() - e).abs().max())
        et = float((t.float() - e).abs().max())
        assert ea <= 1.25 * et + 2e-3, f"{shape} d{n}: ours {ea:.4f} vs torch {et:.4f}"


@pytest.mark.parametrize("shape", [(1, 8, 2, 64, 80, 64, True), (1, 8, 1, 80, 64, 32, True),
                                   (1, 4, 2, 2048, 2048, 32, True)])
def test_bf16_gradients_no_worse_than_torch(shape):
    """bf16 error of the HIP backward vs fp32 stays within PyTorch's own bf16
    SDPA backward error on the same inputs (x1.25 + 2e-3)."""
    b, hq, hkv, sq, sk, d, causal = shape
    q = seeded((b, hq, sq, d), 12, dtype=BF16)
    k = seeded((b, hkv, sk, d), 13, dtype=BF16)
    v = seeded((b, hkv, sk, d), 14, dtype=BF16)
    do = seeded((b, hq, sq, d), 15, dtype=BF16)
    out, lse = attention_forward(q, k, v, causal=causal, scale=1 / math.sqrt(d))
    ours = attention_backward(q, k, v, out, lse, do, causal=causal, scale=1 / math.sqrt(d))
    _, _, exact = reference_fp32(q, k, v, causal=causal, with_grad_out=do)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    g = hq // hkv
    to = torch.nn.functional.scaled_dot_product_attention(
        qq, kk.repeat_interleave(g, 1), vv.repeat_interleave(g, 1), is_causal=causal)
    theirs = torch.autograd.grad(to, (qq, kk, vv), do)
    bar = dict(atol=1e-2, rtol=1e-2)
    for a, t, e, n in zip(ours, theirs, exact, "qkv"):
        ea = float((a.float() - e).abs().max())
        et = float((t.float() - e).abs().max())
        print(f"BF16_VS_TORCH {shape} d{n}: hip {error_stats(a, e, **bar)} "
              f"torch {error_stats(t, e, **bar)}", flush=True)
        assert ea <= 1.25 * et + 2e-3, f"d{n}: ours {ea:.4f} vs torch {et:.4f}"


def test_backward_stages_called_separately():
    """The stage mask of kf_attn_bwd_stages: the row deltas from the delta
    kernel (the dK/dV stage run without dQ in the same call), then dQ, dK/dV
    and the fixup as separate calls, agree with fp32 autograd."""
    from kotflash_amd import _hip
    q = seeded((2, 4, 300, 64), 91, dtype=F16, scale=0.5)
    k = seeded((2, 2, 300, 64), 92, dtype=F16, scale=0.5)
    v = seeded((2, 2, 300, 64), 93, dtype=F16, scale=0.5)
    do = seeded((2, 4, 300, 64), 94, dtype=F16)
    out, lse = attention_forward(q, k, v, causal=True, scale=0.125)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(_hip.bwd_workspace_bytes(2, 4, 2, 300, 300, 64, True), device="cuda",
                     dtype=torch.uint8)
    for st in (_hip.KF_BWD_DELTA, _hip.KF_BWD_DKDV, _hip.KF_BWD_DKDV_FIXUP, _hip.KF_BWD_DQ):
        _hip.bwd(q, k, v, out, lse, do, dq, dk, dv, causal=True, scale=0.125, workspace=ws,
                 stages=st)
    _, _, (eq, ek, ev) = reference_fp32(q, k, v, causal=True, with_grad_out=do)
    assert_close(dq, eq, **BWD_TOL[F16], what="dQ")
    assert_close(dk, ek, **BWD_TOL[F16], what="dK")
    assert_close(dv, ev, **BWD_TOL[F16], what="dV")


def test_config3_bf16_gradients_at_stated_bar():
    """BASELINE config 3 in bf16 at the bar the build target states for
    gradients, in its relative form for bf16: |got - ref| <= 1e-2 + 1e-2 |ref|
    element-wise for dQ, dK and dV (|dV| reaches ~9 here, where one bf16
    half-ulp is 0.031, so an absolute-only 1e-2 cannot hold for any bf16
    output). Prints per-tensor max-abs / max-rel errors and the out-of-bound
    count, next to the same figures for PyTorch's own bf16 SDPA backward
    (flash or memory-efficient kernel, no math path) on identical inputs."""
    import json

    from torch.nn.attention import SDPBackend, sdpa_kernel

    bar = dict(atol=1e-2, rtol=1e-2)
    q = seeded((2, 16, 4096, 128), 301, dtype=BF16, scale=0.5)
    k = seeded((2, 4, 4096, 128), 302, dtype=BF16, scale=0.5)
    v = seeded((2, 4, 4096, 128), 303, dtype=BF16, scale=0.5)
    do = seeded((2, 16, 4096, 128), 304, dtype=BF16)
    out, lse = attention_forward(q, k, v, causal=True, scale=1 / math.sqrt(128))
    ours = attention_backward(q, k, v, out, lse, do, causal=True, scale=1 / math.sqrt(128))
    eo, el, exact = reference_fp32(q, k, v, causal=True, with_grad_out=do)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        to = torch.nn.functional.scaled_dot_product_attention(
            qq, kk.repeat_interleave(4, 1).contiguous(), vv.repeat_interleave(4, 1).contiguous(),
            is_causal=True)
        theirs = torch.autograd.grad(to, (qq, kk, vv), do)
    report = {"bar": "1e-2 + 1e-2 |ref|", "hip": {}, "torch_sdpa_bf16": {}}
    report["hip"]["O"] = error_stats(out, eo, **FWD_TOL[BF16])
    report["torch_sdpa_bf16"]["O"] = error_stats(to, eo, **FWD_TOL[BF16])
    for n, a, t, e in zip(("dQ", "dK", "dV"), ours, theirs, exact):
        report["hip"][n] = error_stats(a, e, **bar)
        report["torch_sdpa_bf16"][n] = error_stats(t, e, **bar)
    print("CONFIG3_BF16_BAR " + json.dumps(report), flush=True)
    assert_close(out, eo, **FWD_TOL[BF16], what="cfg3 bf16 O")
    assert_close(lse, el, **FWD_TOL[BF16], what="cfg3 bf16 LSE")
    for n, a, e in zip(("dQ", "dK", "dV"), ours, exact):
        assert_close(a, e, **bar, what=f"cfg3 bf16 {n} at 1e-2 + 1e-2 |ref|")


def test_long_sequence_training_step():
    """A 16K-token causal GQA step (B=1, Hq=4, Hkv=1, D=128, fp16): 128 key
    tiles, stream-K shares across many tile rows, against fp32 autograd
    (q/k/v scaled 0.5 as in config 3)."""
    s, d = 16384, 128
    q = seeded((1, 4, s, d), 1901, dtype=F16, scale=0.5)
    k = seeded((1, 1, s, d), 1902, dtype=F16, scale=0.5)
    v = seeded((1, 1, s, d), 1903, dtype=F16, scale=0.5)
    do = seeded((1, 4, s, d), 1904, dtype=F16)
    _check_grads(q, k, v, do, True, F16, "S=16384")
