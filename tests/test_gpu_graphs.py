"""HIP-graph capture of the launch paths: each graph is replayed several
times with new inputs written eagerly between replays (and synchronizations),
and every replay is checked against an eager run on the same inputs. The
kernels are deterministic, so replays must match bit for bit."""
import pytest
import torch

import kotflash_amd as kf
from kotflash_amd import _hip
from tests.gpu_helpers import seeded

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _capture(fn):
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()  # warm-up outside the graph (plans, allocator pools)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            result = fn()
    torch.cuda.synchronize()
    return graph, result


def test_public_decode_graph_replays():
    q = seeded((2, 8, 1, 64), 1201, dtype=F16)
    k = seeded((2, 2, 4096, 64), 1202, dtype=F16)
    v = seeded((2, 2, 4096, 64), 1203, dtype=F16)
    graph, out = _capture(lambda: kf.attention(q, k, v, causal=False, backend="hip"))
    for r in range(3):
        q.copy_(seeded(q.shape, 1300 + r, dtype=F16))
        k.copy_(seeded(k.shape, 1310 + r, dtype=F16))
        v.copy_(seeded(v.shape, 1320 + r, dtype=F16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = kf.attention(q, k, v, causal=False, backend="hip")
        assert torch.equal(out, expected), f"replay {r}"


@pytest.mark.parametrize("causal", [True, False])
def test_forward_backward_graph_replays(causal):
    b, hq, hkv, s, d = 1, 8, 2, 700, 128
    q, k, v, do = (torch.empty(sh, dtype=F16, device="cuda") for sh in
                   ((b, hq, s, d), (b, hkv, s, d), (b, hkv, s, d), (b, hq, s, d)))
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, s), dtype=torch.float32, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(_hip.bwd_workspace_bytes(b, hq, hkv, s, s, d, causal), dtype=torch.uint8,
                     device="cuda")

    def step():
        _hip.fwd(q, k, v, out, lse, causal=causal, scale=0.09)
        _hip.bwd(q, k, v, out, lse, do, dq, dk, dv, causal=causal, scale=0.09, workspace=ws)

    for t, seed in zip((q, k, v, do), (1401, 1402, 1403, 1404)):
        t.copy_(seeded(t.shape, seed, dtype=F16))
    graph, _ = _capture(step)
    for r in range(3):
        for t, seed in zip((q, k, v, do), (1500, 1510, 1520, 1530)):
            t.copy_(seeded(t.shape, seed + r, dtype=F16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [x.clone() for x in (out, lse, dq, dk, dv)]
        step()  # eager on the same inputs
        torch.cuda.synchronize()
        for name, g, e in zip(("O", "LSE", "dQ", "dK", "dV"), got, (out, lse, dq, dk, dv)):
            assert torch.equal(g, e), f"replay {r}: {name}"


def test_ragged_append_and_decode_graph_replays():
    b, hkv, hq, cap, d, n = 3, 2, 8, 4096, 64, 2
    lengths = [1500, 3000, 2200]
    kc = torch.full((b, hkv, cap, d), float("nan"), dtype=F16, device="cuda")
    vc = torch.full_like(kc, float("nan"))
    for i, L in enumerate(lengths):
        kc[i, :, :L] = seeded((hkv, L, d), 1600 + i, dtype=F16)
        vc[i, :, :L] = seeded((hkv, L, d), 1610 + i, dtype=F16)
    starts = torch.tensor(lengths, dtype=torch.int64, device="cuda")
    seqlens = torch.tensor([L + n for L in lengths], dtype=torch.int32, device="cuda")
    maxlen = max(lengths) + n
    nk = torch.empty((b, hkv, n, d), dtype=F16, device="cuda")
    nv = torch.empty_like(nk)
    q = torch.empty((b, hq, n, d), dtype=F16, device="cuda")
    out = torch.empty_like(q)
    splits = _hip.decode_num_splits_ragged(b, hq, hkv, n, [L + n for L in lengths], d)
    ws = torch.empty(max(256, _hip.decode_workspace_bytes(b, hq, hkv, n, d, splits)),
                     dtype=torch.uint8, device="cuda")

    def step():
        _hip.kv_append(kc, vc, nk, nv, start_dev=starts, max_start=max(lengths))
        _hip.decode(q, kc[:, :, :maxlen], vc[:, :, :maxlen], out, None, seqlens, scale=0.125,
                    num_splits=splits, workspace=ws)

    for t, seed in zip((nk, nv, q), (1701, 1702, 1703)):
        t.copy_(seeded(t.shape, seed, dtype=F16))
    graph, _ = _capture(step)
    for r in range(3):
        for t, seed in zip((nk, nv, q), (1800, 1810, 1820)):
            t.copy_(seeded(t.shape, seed + r, dtype=F16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        step()
        torch.cuda.synchronize()
        assert torch.equal(got, out), f"replay {r}: O"
        for i, L in enumerate(lengths):
            assert torch.equal(kc[i, :, L:L + n], nk[i]) and torch.equal(vc[i, :, L:L + n], nv[i])
        assert bool(torch.isfinite(out).all())


def test_fused_append_decode_graph_replays():
    """kf_attn_append_decode captured in a graph: each replay stores the new
    tokens (written eagerly before it) and decodes; every replay matches an
    eager call on the same inputs bit for bit, cache included."""
    b, hkv, hq, cap, d, n = 3, 2, 8, 4096, 64, 3
    lengths = [0, 2900, 1400]
    kc = torch.full((b, hkv, cap, d), float("nan"), dtype=F16, device="cuda")
    vc = torch.full_like(kc, float("nan"))
    for i, L in enumerate(lengths):
        if L:
            kc[i, :, :L] = seeded((hkv, L, d), 1900 + i, dtype=F16)
            vc[i, :, :L] = seeded((hkv, L, d), 1910 + i, dtype=F16)
    seqlens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    nk = torch.empty((b, hkv, n, d), dtype=F16, device="cuda")
    nv = torch.empty_like(nk)
    q = torch.empty((b, hq, n, d), dtype=F16, device="cuda")
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, n), dtype=torch.float32, device="cuda")
    splits = _hip.decode_num_splits_ragged(b, hq, hkv, n, lengths, d)
    ws = torch.empty(_hip.decode_workspace_bytes(b, hq, hkv, n, d, splits + 1),
                     dtype=torch.uint8, device="cuda")

    def step():
        _hip.append_decode(q, kc, vc, nk, nv, out, lse, seqlens, past_length=0,
                           max_length=max(lengths), scale=0.125, num_splits=splits, workspace=ws)

    for t, seed in zip((nk, nv, q), (1921, 1922, 1923)):
        t.copy_(seeded(t.shape, seed, dtype=F16))
    graph, _ = _capture(step)
    for r in range(3):
        for t, seed in zip((nk, nv, q), (1930, 1940, 1950)):
            t.copy_(seeded(t.shape, seed + r, dtype=F16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got, got_lse = out.clone(), lse.clone()
        for i, L in enumerate(lengths):
            assert torch.equal(kc[i, :, L:L + n], nk[i]) and torch.equal(vc[i, :, L:L + n], nv[i])
            assert torch.isnan(kc[i, :, L + n:]).all()
        step()
        torch.cuda.synchronize()
        assert torch.equal(got, out) and torch.equal(got_lse, lse), f"replay {r}"
        assert bool(torch.isfinite(out).all())


def test_decode_workspaces_per_stream_and_fresh_under_capture():
    """The eager decode reuses one workspace per (device, stream): calls on
    two streams at once must not share it, and a graph captured on one
    stream must hold its own workspace, so replaying it on another stream
    while eager calls run on the capturing stream races with nothing."""
    q1 = seeded((2, 8, 1, 64), 1701, dtype=F16)
    k1 = seeded((2, 2, 8192, 64), 1702, dtype=F16)
    v1 = seeded((2, 2, 8192, 64), 1703, dtype=F16)
    q2 = seeded((2, 8, 1, 64), 1711, dtype=F16)
    k2 = seeded((2, 2, 8192, 64), 1712, dtype=F16)
    v2 = seeded((2, 2, 8192, 64), 1713, dtype=F16)
    ref1 = kf.attention(q1, k1, v1, causal=False, backend="hip")
    ref2 = kf.attention(q2, k2, v2, causal=False, backend="hip")
    assert not torch.equal(ref1, ref2)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    for r in range(3):
        with torch.cuda.stream(sa):
            oa = kf.attention(q1, k1, v1, causal=False, backend="hip")
        with torch.cuda.stream(sb):
            ob = kf.attention(q2, k2, v2, causal=False, backend="hip")
        torch.cuda.synchronize()
        assert torch.equal(oa, ref1) and torch.equal(ob, ref2), f"two streams, round {r}"
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(sa):
        with torch.cuda.graph(graph, stream=sa):
            gout = kf.attention(q1, k1, v1, causal=False, backend="hip")
    torch.cuda.synchronize()
    for r in range(3):
        with torch.cuda.stream(sb):
            graph.replay()
        with torch.cuda.stream(sa):
            eager = kf.attention(q2, k2, v2, causal=False, backend="hip")
        torch.cuda.synchronize()
        assert torch.equal(gout, ref1), f"replay {r}"
        assert torch.equal(eager, ref2), f"eager beside replay {r}"
