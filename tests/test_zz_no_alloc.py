"""kf_attn_decode_noalloc against kf_attn_decode, through the C ABI.

The allocation-free decode has no counterpart in the reference; it serves
callers that cannot allocate device memory. Its split partials live in the
library's static per-device scratch instead of a workspace. For the same
split count it runs the same kernels in the same order, so its O and LSE must
be bit-identical to the workspace entry point's, and both must match dense
fp32 attention within the fp16 tolerance. The two calls run back to back,
the second on a smaller problem, which then reads a scratch that still holds
the first call's partials beyond its own.
"""
import math

import pytest
import torch

from kotflash_amd import _hip
from tests.gpu_helpers import FWD_TOL, assert_close, reference_fp32, seeded

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _both_paths(q, k, v, seqlens, host_lengths):
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    if host_lengths is None:
        splits = _hip.decode_num_splits(b, hq, hkv, sq, sk, d)
    else:
        splits = _hip.decode_num_splits_ragged(b, hq, hkv, sq, host_lengths, d)
    assert splits > 1  # the partials (and so the scratch) are used
    scale = 1.0 / math.sqrt(d)
    o_ws, o_na = torch.empty_like(q), torch.full_like(q, float("nan"))
    l_ws = torch.empty((b, hq, sq), device="cuda", dtype=torch.float32)
    l_na = torch.full_like(l_ws, float("nan"))
    ws = torch.empty(_hip.decode_workspace_bytes(b, hq, hkv, sq, d, splits), device="cuda",
                     dtype=torch.uint8)
    _hip.decode(q, k, v, o_ws, l_ws, seqlens, scale=scale, num_splits=splits, workspace=ws)
    _hip.decode_noalloc(q, k, v, o_na, l_na, seqlens, scale=scale, num_splits=splits)
    torch.cuda.synchronize()
    return splits, (o_ws, l_ws), (o_na, l_na)


def test_noalloc_decode_matches_workspace_decode_on_two_calls():
    # Call 1: BASELINE config 2 at Sk = 16384 (64 splits).
    print("noalloc call 1: B=2 Hq=8 Hkv=2 Sq=1 Sk=16384 D=64 fp16", flush=True)
    q = seeded((2, 8, 1, 64), 9801, dtype=F16)
    k = seeded((2, 2, 16384, 64), 9802, dtype=F16)
    v = seeded((2, 2, 16384, 64), 9803, dtype=F16)
    splits1, (o1, l1), (n1, m1) = _both_paths(q, k, v, None, None)
    assert torch.equal(o1, n1) and torch.equal(l1, m1)
    eo, el = reference_fp32(q, k, v, causal=False)
    assert_close(n1, eo, **FWD_TOL[F16], what="noalloc O, call 1")
    assert_close(m1, el, **FWD_TOL[F16], what="noalloc LSE, call 1")
    # Call 2, smaller: one sequence, 4 query rows, ragged visible lengths.
    print("noalloc call 2: B=2 Hq=4 Hkv=1 Sq=3 Sk=3000 D=64 fp16, lengths [2500, 3000]",
          flush=True)
    q = seeded((2, 4, 3, 64), 9804, dtype=F16)
    k = seeded((2, 1, 3000, 64), 9805, dtype=F16)
    v = seeded((2, 1, 3000, 64), 9806, dtype=F16)
    lengths = [2500, 3000]
    seqlens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    splits2, (o2, l2), (n2, m2) = _both_paths(q, k, v, seqlens, lengths)
    assert splits2 < splits1
    assert torch.equal(o2, n2) and torch.equal(l2, m2)
    for i, n in enumerate(lengths):
        eo, el = reference_fp32(q[i:i + 1], k[i:i + 1, :, :n], v[i:i + 1, :, :n], causal=False)
        assert_close(n2[i:i + 1], eo, **FWD_TOL[F16], what=f"noalloc O, call 2, seq {i}")
        assert_close(m2[i:i + 1], el, **FWD_TOL[F16], what=f"noalloc LSE, call 2, seq {i}")


_CAPTURE_CHILD = r'''
import math, sys
sys.path.insert(0, sys.argv[1])
import torch
from kotflash_amd import _hip
from tests.gpu_helpers import seeded
torch.cuda.set_device(0)
b, hq, hkv, sq, sk, d = 2, 8, 2, 1, 16384, 64
scale = 1.0 / math.sqrt(d)
splits = _hip.decode_num_splits(b, hq, hkv, sq, sk, d)
q, k, v = (torch.empty(s, device="cuda", dtype=torch.float16)
           for s in ((b, hq, sq, d), (b, hkv, sk, d), (b, hkv, sk, d)))
o, lse = torch.empty_like(q), torch.empty((b, hq, sq), device="cuda", dtype=torch.float32)
# Warm-up on a side stream, as torch.cuda.graph expects: the workspace entry
# point only, so the no-alloc entry point's first call of this process (and its
# per-device scratch lookup) happens inside the capture below.
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side):
    ws = torch.empty(_hip.decode_workspace_bytes(b, hq, hkv, sq, d, splits), device="cuda",
                     dtype=torch.uint8)
    _hip.decode(q.zero_(), k.zero_(), v.zero_(), o, lse, None, scale=scale, num_splits=splits,
                workspace=ws)
torch.cuda.current_stream().wait_stream(side)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
print("capturing the first kf_attn_decode_noalloc call", flush=True)
with torch.cuda.graph(g):
    _hip.decode_noalloc(q, k, v, o, lse, None, scale=scale, num_splits=splits)
print("captured", flush=True)
for r in range(3):
    q.copy_(seeded((b, hq, sq, d), 9900 + r, dtype=torch.float16))
    k.copy_(seeded((b, hkv, sk, d), 9910 + r, dtype=torch.float16))
    v.copy_(seeded((b, hkv, sk, d), 9920 + r, dtype=torch.float16))
    # Eager work between replays, including an eager no-alloc call on other
    # inputs, which overwrites the shared scratch the graph's kernels use.
    q2 = seeded((1, 4, 2, d), 9930 + r, dtype=torch.float16)
    k2 = seeded((1, 1, 3000, d), 9940 + r, dtype=torch.float16)
    o2 = torch.empty_like(q2)
    _hip.decode_noalloc(q2, k2, k2, o2, None, None, scale=scale,
                        num_splits=_hip.decode_num_splits(1, 4, 1, 2, 3000, d))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    eo, el = torch.empty_like(o), torch.empty_like(lse)
    _hip.decode(q, k, v, eo, el, None, scale=scale, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(o, eo) and torch.equal(lse, el), f"replay {r} differs from kf_attn_decode"
    print(f"replay {r} bit-identical", flush=True)
print("CHILD_OK", flush=True)
'''


def test_noalloc_first_call_inside_graph_capture():
    """The use case the entry point exists for: its first call in a process
    (which resolves the device's scratch address) made under HIP graph
    capture. A fresh process captures that call into a torch CUDA graph,
    replays it three times with eager work in between (an eager no-alloc call
    on other inputs overwrites the scratch each time), and every replay must
    be bit-identical to kf_attn_decode with a workspace on the same inputs."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    print("noalloc capture child: B=2 Hq=8 Hkv=2 Sq=1 Sk=16384 D=64 fp16", flush=True)
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True,
                         text=True, timeout=100)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "CHILD_OK" in res.stdout
