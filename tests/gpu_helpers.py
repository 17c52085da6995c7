"""Shared helpers of the GPU parity tests."""
import math

import torch

# Tolerances against fp32 references. O/LSE: atol = rtol = 2e-3 for fp16 and
# 1e-2 for bf16; fp16 gradients: atol 1e-2 (the build target's figures).
# bf16 gradients: atol 3e-2 + rtol 1e-2. P and dS are rounded to the input
# dtype before their products (as in the reference, triton_backward.py:85,
# :183-184), and with bf16's 8-bit mantissa that alone moves dK/dV by up to
# 3e-2 at these shapes: PyTorch's own bf16 SDPA backward on identical inputs
# measured 2.6e-2 (Hq=8, Hkv=2, S=64/80) and 3.2e-2 (B=2, Hq=16, S=4096, where
# |dV| reaches 9.8 and one bf16 half-ulp is 0.031) against the same fp32
# reference. test_bf16_gradients_no_worse_than_torch checks that relation.
FWD_TOL = {torch.float16: dict(atol=2e-3, rtol=2e-3), torch.bfloat16: dict(atol=1e-2, rtol=1e-2)}
BWD_TOL = {torch.float16: dict(atol=1e-2, rtol=0.0), torch.bfloat16: dict(atol=3e-2, rtol=1e-2)}


def seeded(shape, seed, *, dtype, scale=1.0, device="cuda"):
    """Seeded N(0,1)*scale on the CPU, rounded to dtype, then moved to the GPU
    so the CPU oracle and the GPU see identical values."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(device)


def reference_fp32(q, k, v, *, causal, scale=None, with_grad_out=None):
    """Dense fp32 attention on K/V expanded to Hq heads: (O, LSE) and,
    with ``with_grad_out``, (dq, dk, dv) by autograd (summed over GQA groups)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    group = q.shape[1] // k.shape[1]
    qf, kf, vf = (t.detach().float().clone().requires_grad_(with_grad_out is not None)
                  for t in (q, k, v))
    ke = kf.repeat_interleave(group, dim=1)
    ve = vf.repeat_interleave(group, dim=1)
    s = torch.matmul(qf, ke.transpose(-2, -1).contiguous()) * scale
    if causal:
        i = torch.arange(q.shape[2], device=q.device)[:, None]
        j = torch.arange(k.shape[2], device=q.device)[None, :]
        s = s.masked_fill(j > i, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    out = torch.matmul(torch.softmax(s, dim=-1), ve)
    if with_grad_out is None:
        return out.detach(), lse.detach()
    grads = torch.autograd.grad(out, (qf, kf, vf), with_grad_out.float())
    return out.detach(), lse.detach(), grads


def assert_close(actual, expected, *, atol, rtol, what=""):
    a = actual.float()
    e = expected.float().to(a.device)
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    bad = err > bound
    if bool(bad.any()) or not bool(torch.isfinite(a).all()):
        idx = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {a.numel()} elements out of tolerance "
            f"(atol={atol}, rtol={rtol}); max abs err {float(err.max()):.3e}; worst at flat "
            f"index {idx}: got {float(a.flatten()[idx]):.6f} want {float(e.flatten()[idx]):.6f}"
        )
