"""bf16 gradients at the stated bar, case by case, with the figures that say
where each miss comes from.

The bar is the build target's gradient tolerance in the relative form bf16
needs: |got - ref| <= 1e-2 + 1e-2 |ref| against exact fp32 autograd on the
same bf16-rounded inputs. For every bf16 backward case of the GPU suite (the
reference's backward cases, tests/test_triton.py:160-174, run in bf16; the
split-dQ shapes; the seeded random shapes) the test prints
one line of per-tensor figures (max abs error, max relative error where
|ref| >= 1e-2, elements outside the bar) for three computations:

* ``hip``: this build's kernels;
* ``ref_alg``: the reference kernels' own arithmetic at bf16 precision (P and
  dS rounded to bf16 before their products, reference
  kotflash/kernels/triton_backward.py:85,183-184; tests/gpu_helpers.py
  reference_algorithm_rounded), dense in fp32;
* ``torch``: PyTorch's bf16 SDPA backward.

A case passes when the HIP result has no element outside the bar, or when it
is one of the named exceptions below: there the reference's own algorithm at
bf16 (or PyTorch's bf16 backward) misses the bar on the same inputs too, so
the miss is the bf16 rounding of P and dS that the reference also does, and
the HIP error must stay within 1.25x of theirs + 2e-3. ``hip_vs_ref_alg`` (the
largest difference between the two) shows that the HIP kernels implement that
arithmetic.
"""
import json
import math
import random

import pytest
import torch

from kotflash_amd.kernels.hip_backward import attention_backward
from kotflash_amd.kernels.hip_forward import attention_forward
from tests.gpu_helpers import error_stats, reference_algorithm_rounded, reference_fp32, seeded

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
BAR = dict(atol=1e-2, rtol=1e-2)


def _random_bf16_shapes(n=12, seed=4202):
    # The shapes of tests/test_gpu_random_shapes.py::test_random_shape_bf16.
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        hkv = rng.choice([1, 2, 3, 4])
        hq = hkv * rng.choice([1, 2, 4, 8])
        b = rng.choice([1, 2, 3])
        sq = rng.randint(1, 2500)
        sk = sq if rng.random() < 0.5 else rng.randint(1, 2500)
        d = rng.choice([8, 16, 40, 64, 72, 80, 96, 104, 128])
        out.append((b, hq, hkv, sq, sk, d, rng.random() < 0.5))
    return out


# (name, (B, Hq, Hkv, Sq, Sk, D, causal), seeds of q, k, v, dO, input scale)
CASES = [
    *[(f"ref{i}", (1,) + s, (12, 13, 14, 15), 1.0) for i, s in enumerate([
        (4, 4, 64, 80, 32, False), (8, 2, 64, 80, 64, True), (8, 1, 80, 64, 32, True),
        (8, 2, 48, 64, 72, False), (4, 4, 48, 64, 96, True), (8, 1, 64, 48, 128, False),
        (8, 2, 1024, 1024, 64, True), (4, 1, 1024, 768, 32, False),
        (4, 2, 2048, 2048, 32, True), (8, 2, 1, 1024, 64, False)])],
    ("split_dq0", (1, 2, 1, 2500, 700, 128, True), (89, 90, 91, 92), 1.0),
    ("split_dq1", (2, 16, 4, 512, 512, 96, True), (89, 90, 91, 92), 1.0),
    *[(f"rand{i}", s, (511, 512, 513, 514), 1.0) for i, s in enumerate(_random_bf16_shapes())],
    ("config3", (2, 16, 4, 4096, 4096, 128, True), (301, 302, 303, 304), 0.5),
]

# Named exceptions (case, tensor), measured on MI355X: the HIP result misses
# the bar on as many elements as the reference's algorithm at bf16 does on the
# same inputs (PyTorch's bf16 backward misses on as many or more):
#   ref1 dV       hip 1 (max abs 0.0192), ref_alg 1 (0.0176), torch 1 (0.0256)
#   split_dq1 dK  hip 1 (0.0196),         ref_alg 1 (0.0190), torch 7 (0.0225)
#   rand0 dV      hip 2 (0.0294),         ref_alg 2 (0.0443), torch 10 (0.0353)
EXCEPTIONS = {("ref1", "dV"), ("split_dq1", "dK"), ("rand0", "dV")}


@pytest.mark.parametrize("name,shape,seeds,scl", CASES, ids=[c[0] for c in CASES])
def test_bf16_gradients_at_bar(name, shape, seeds, scl):
    b, hq, hkv, sq, sk, d, causal = shape
    print(f"bf16 bar case {name}: {shape}", flush=True)
    q = seeded((b, hq, sq, d), seeds[0], dtype=BF16, scale=scl)
    k = seeded((b, hkv, sk, d), seeds[1], dtype=BF16, scale=scl)
    v = seeded((b, hkv, sk, d), seeds[2], dtype=BF16, scale=scl)
    do = seeded((b, hq, sq, d), seeds[3], dtype=BF16)
    scale = 1 / math.sqrt(d)
    out, lse = attention_forward(q, k, v, causal=causal, scale=scale)
    ours = attention_backward(q, k, v, out, lse, do, causal=causal, scale=scale)
    _, _, exact = reference_fp32(q, k, v, causal=causal, scale=scale, with_grad_out=do)
    alg = reference_algorithm_rounded(q, k, v, do, causal=causal, scale=scale)[1:]
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    g = hq // hkv
    to = torch.nn.functional.scaled_dot_product_attention(
        qq, kk.repeat_interleave(g, 1).contiguous(), vv.repeat_interleave(g, 1).contiguous(),
        is_causal=causal, scale=scale)
    theirs = torch.autograd.grad(to, (qq, kk, vv), do)
    report, failures = {"case": name, "shape": shape}, []
    for n, a, r, t, e in zip(("dQ", "dK", "dV"), ours, alg, theirs, exact):
        fig = {"hip": error_stats(a, e, **BAR), "ref_alg": error_stats(r, e, **BAR),
               "torch": error_stats(t, e, **BAR),
               "hip_vs_ref_alg": float((a.float() - r).abs().max())}
        report[n] = fig
        if fig["hip"]["outside"] == 0:
            continue
        # A named exception stays one only while the reference's algorithm at
        # bf16 (or torch) misses on at least as many elements and the HIP
        # error stays within 1.25x of theirs + 2e-3.
        most = max(fig["ref_alg"]["outside"], fig["torch"]["outside"])
        limit = 1.25 * max(fig["ref_alg"]["max_abs"], fig["torch"]["max_abs"]) + 2e-3
        if ((name, n) not in EXCEPTIONS or fig["hip"]["outside"] > most
                or fig["hip"]["max_abs"] > limit):
            failures.append(f"{n}: {fig['hip']['outside']} outside the bar "
                            f"(ref_alg {fig['ref_alg']['outside']}, torch {fig['torch']['outside']})")
    print("BF16_BAR " + json.dumps(report), flush=True)
    assert not failures, f"{name} {shape}: " + "; ".join(failures)
