#!/usr/bin/env python3
"""Headline benchmark of the kotflash_amd attention hot path on one MI355X.

One JSON line on stdout (everything else goes to stderr):

* ``value``: causal GQA fwd+bwd TFLOP/s at BASELINE config 3 (B=2, Hq=16,
  Hkv=4, S=4096, D=128, fp16, q/k/v ~ 0.5 N(0,1), dO ~ N(0,1)). A step is one
  forward plus one backward (4 launches: forward, dQ with the row deltas,
  dK/dV, dK/dV fixup) on
  inputs already resident in HBM; exactly ``--steps`` steps are timed between
  two ``torch.cuda.synchronize()``. Work per step is the algorithmic
  4.8115e11 FLOP (forward 4 D B Hq S(S+1)/2, backward 2.5x that).
* ``roofline``: the dominant kernel (the dK/dV kernel), its algorithmic
  FLOP per launch (the 4 of the 5 backward GEMMs it computes:
  S = Q K^T, dP = dO V^T, dV, dK = 2x the forward FLOP = 2.7494e11) over its
  average launch time, from HIP events recorded around it on its launch
  stream in a second pass of as many identical steps right after the timed
  ones (the events add about 6 us to a step, so the timed steps carry none);
  peak = MI355X dense fp16 MFMA 2.5 PFLOP/s.
  ``traffic`` is the HBM bytes per dK/dV launch read from rocprofv3
  FETCH_SIZE + WRITE_SIZE counters (profiles/), calibrated on a copy kernel.
* ``kernels``: every launch of the step timed on its own, 20 back-to-back
  launches between two events, after the timed steps.
* ``decode``: BASELINE config 2 at Sk=16384 (B=2, Hq=8, Hkv=2, Sq=1, D=64,
  fp16): microseconds per call (split-KV kernel + LSE merge) from HIP-graph
  replays of back-to-back calls over 32 rotating K/V sets (537 MB, larger than
  the 256 MB Infinity Cache), the median of 5 timed batches of replays, and
  HBM GB/s of the 16,781,376 algorithmic bytes.
* ``configs``: the other BASELINE configurations timed on the GPU: config 1
  (forward only), config 2 over Sk in {2048, 4096, 8192, 16384}, config 3 in
  bf16, config 4 (non-causal MHA fwd+bwd, D = 72 and 96) and config 5 (64
  steps of per-sequence KV append + ragged split-KV decode on a
  [8, 8, 32768, 64] cache), each with its own roofline fraction.
* ``cpu_baseline``: the reference's SDPA path (native-GQA
  scaled_dot_product_attention, fp32, autograd backward) on the host CPU at the
  full config 3 shape, median of 5 timed steps after one warm-up.

``--gpus N`` with N > 1 exits with status 2: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

METRIC = "fwd+bwd TFLOP/s at S=4096,D=128; split-KV decode µs/token + HBM GB/s"
CFG3 = dict(B=2, Hq=16, Hkv=4, S=4096, D=128)
CFG2 = dict(B=2, Hq=8, Hkv=2, Sq=1, Sk=16384, D=64)
PEAK_MFMA_F16 = 2.5e15
PEAK_HBM = 8.0e12
# HBM-side bytes per dK/dV launch at config 3 fp16: rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE of the warm dK/dV dispatch of `bench.py --pmc-sample`, each scaled by the
# factor the same counter reads for a 512 MiB copy / fill in that program
# (profiles/dkdv_cfg3_hbm_traffic.md). Re-measure when the dK/dV kernel changes.
DKDV_TRAFFIC_BYTES = 1.531e8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def fwd_flops(b, hq, s, d):
    return 4.0 * d * b * hq * s * (s + 1) / 2.0


def seeded(torch, shape, seed, dtype, scale=1.0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(device)


# An idle MI355X raises its clocks over the first ~30 ms of MFMA load: from a
# cold start the config 3 step measured 3.47 ms (first launch), then 0.68 to
# 0.86 ms over steps 1-20 and a steady 0.665 ms from step ~40 on. Steps of a
# training loop run back to back, so the figure is taken at the steady
# state: untimed steps run for PREWARM_MS of wall time before the --warmup
# steps, and the JSON line states how many.
PREWARM_MS = 200.0


def prewarm(torch, fn, ms):
    """Run ``fn`` untimed until ``ms`` milliseconds of wall time have passed
    (checked every 10 calls, after a synchronize); returns the call count."""
    if ms <= 0:
        return 0
    n = 0
    t0 = time.perf_counter()
    while True:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= ms:
            return n


def bench_train(torch, _hip, dtype, steps, warmup, cfg=None, causal=True, qkv_scale=0.5,
                prewarm_ms=PREWARM_MS):
    c = cfg or CFG3
    b, hq, hkv, s, d = c["B"], c["Hq"], c["Hkv"], c["S"], c["D"]
    scale = 1.0 / math.sqrt(d)
    q = seeded(torch, (b, hq, s, d), 301, dtype, qkv_scale)
    k = seeded(torch, (b, hkv, s, d), 302, dtype, qkv_scale)
    v = seeded(torch, (b, hkv, s, d), 303, dtype, qkv_scale)
    do = seeded(torch, (b, hq, s, d), 304, dtype)
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, s), device=q.device, dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(_hip.bwd_workspace_bytes(b, hq, hkv, s, s, d, causal), device=q.device,
                     dtype=torch.uint8)

    def fwd():
        _hip.fwd(q, k, v, out, lse, causal=causal, scale=scale)

    def bwd(stages):
        _hip.bwd(q, k, v, out, lse, do, dq, dk, dv, causal=causal, scale=scale,
                 workspace=ws, stages=stages)

    def step(ev=None):
        fwd()
        bwd(_hip.KF_BWD_DELTA | _hip.KF_BWD_DQ)  # dQ kernel (computes the row deltas too)
        if ev is not None:
            ev[0].record()
        bwd(_hip.KF_BWD_DKDV)
        if ev is not None:
            ev[1].record()
        bwd(_hip.KF_BWD_DKDV_FIXUP)

    # The launches go to torch's current stream, so events recorded on it
    # bracket exactly the dK/dV kernel inside a step. torch creates the HIP
    # event on its first record; recording every event once here keeps that
    # creation out of the measured steps.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for e in [start, stop] + [x for pair in evs for x in pair]:
        e.record()
    nwarm = prewarm(torch, step, prewarm_ms)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # The timed steps carry no event between launches: the two events around
    # a dK/dV launch add about 6 us to a config 3 step (1%, measured).
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ms = start.elapsed_time(stop) / steps
    # The dK/dV kernel's live duration: the same number of identical steps
    # right after, with events around every dK/dV launch.
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    dkdv_live = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)

    # Per-kernel figures: each launch repeated back to back between two events
    # (no event between launches), after the timed steps.
    def isolated(fn, n=20):
        fn()
        torch.cuda.synchronize()
        a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        z.record()
        torch.cuda.synchronize()
        return a.elapsed_time(z) / n

    per = {
        "attn_fwd": isolated(fwd),
        "bwd_dq": isolated(lambda: bwd(_hip.KF_BWD_DQ)),
        "bwd_dkdv": isolated(lambda: bwd(_hip.KF_BWD_DKDV)),
        "bwd_dkdv_fixup": isolated(lambda: bwd(_hip.KF_BWD_DKDV_FIXUP)),
    }
    f = fwd_flops(b, hq, s, d) if causal else 4.0 * d * b * hq * s * s
    work = {"attn_fwd": f, "bwd_dq": 0.5 * f, "bwd_dkdv": 2.0 * f, "bwd_dkdv_fixup": 0.0}
    return ms, wall_ms, dkdv_live, per, work, 3.5 * f, nwarm


def pmc_sample(torch, _hip, dtype):
    """Two config 3 steps (forward, delta, dQ, dK/dV, fixup) followed by a
    512 MiB fill and a 512 MiB device copy, for per-dispatch counter runs
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE): the fill and copy have known
    HBM traffic (0 + 512 MiB and 512 + 512 MiB) and calibrate the counters'
    scale for the dK/dV dispatch."""
    c = CFG3
    b, hq, hkv, s, d = c["B"], c["Hq"], c["Hkv"], c["S"], c["D"]
    scale = 1.0 / math.sqrt(d)
    q = seeded(torch, (b, hq, s, d), 301, dtype, 0.5)
    k = seeded(torch, (b, hkv, s, d), 302, dtype, 0.5)
    v = seeded(torch, (b, hkv, s, d), 303, dtype, 0.5)
    do = seeded(torch, (b, hq, s, d), 304, dtype)
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, s), device=q.device, dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(_hip.bwd_workspace_bytes(b, hq, hkv, s, s, d, True), device=q.device,
                     dtype=torch.uint8)
    # The step runs twice; summaries read each kernel's last dispatch. A
    # kernel's first dispatch can carry one-time runtime set-up (the dQ
    # kernel's first launch, for instance, waits for its scratch space).
    for _ in range(2):
        _hip.fwd(q, k, v, out, lse, causal=True, scale=scale)
        for st in (_hip.KF_BWD_DELTA, _hip.KF_BWD_DQ, _hip.KF_BWD_DKDV, _hip.KF_BWD_DKDV_FIXUP):
            _hip.bwd(q, k, v, out, lse, do, dq, dk, dv, causal=True, scale=scale, workspace=ws,
                     stages=st)
    n = 256 << 20
    src = torch.empty(n, device=q.device, dtype=torch.float16)
    dst = torch.empty_like(src)
    src.fill_(1.0)
    dst.copy_(src)
    torch.cuda.synchronize()
    return {"dispatches": ["attn_fwd", "bwd_delta", "bwd_dq", "bwd_dkdv", "bwd_dkdv_fixup"] * 2
            + ["fill 512 MiB", "copy 512 MiB"], "copy_bytes": 2 * n}


def bench_api(torch, kf, dtype, steps, warmup, prewarm_ms=PREWARM_MS):
    """Same step through the public API: attention(backend="hip") + autograd,
    wall time over `steps` steps after the same pre-warm as the kernel
    figure (a short run measures allocator and clock warm-up instead)."""
    c = CFG3
    q = seeded(torch, (c["B"], c["Hq"], c["S"], c["D"]), 301, dtype, 0.5).requires_grad_(True)
    k = seeded(torch, (c["B"], c["Hkv"], c["S"], c["D"]), 302, dtype, 0.5).requires_grad_(True)
    v = seeded(torch, (c["B"], c["Hkv"], c["S"], c["D"]), 303, dtype, 0.5).requires_grad_(True)
    do = seeded(torch, (c["B"], c["Hq"], c["S"], c["D"]), 304, dtype)

    def step():
        out = kf.attention(q, k, v, causal=True, backend="hip")
        torch.autograd.grad(out, (q, k, v), do)

    prewarm(torch, step, prewarm_ms)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


REPLAY_BATCHES = 5


def replay_median_us(torch, graph, replays, calls_per_replay):
    """Microseconds per captured call: the median over REPLAY_BATCHES timed
    batches of `replays` back-to-back replays of `graph`. One batch on a busy
    or re-clocking box has read 2.6x its usual time; the median keeps such a
    batch out of the figure."""
    batches = []
    for _ in range(REPLAY_BATCHES):
        a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(replays):
            graph.replay()
        z.record()
        torch.cuda.synchronize()
        batches.append(a.elapsed_time(z) * 1e3 / (replays * calls_per_replay))
    return statistics.median(batches)


def bench_decode(torch, _hip, dtype, sk, replays=20):
    c = dict(CFG2, Sk=sk)
    b, hq, hkv, sq, d = c["B"], c["Hq"], c["Hkv"], c["Sq"], c["D"]
    nsets = 32
    ks = [seeded(torch, (b, hkv, sk, d), 1000 + i, dtype) for i in range(nsets)]
    vs = [seeded(torch, (b, hkv, sk, d), 2000 + i, dtype) for i in range(nsets)]
    q = seeded(torch, (b, hq, sq, d), 3000, dtype)
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, sq), device=q.device, dtype=torch.float32)
    splits = _hip.decode_num_splits(b, hq, hkv, sq, sk, d)
    ws = torch.empty(max(256, _hip.decode_workspace_bytes(b, hq, hkv, sq, d, splits)), device=q.device,
                     dtype=torch.uint8)

    def calls():
        for i in range(nsets):
            _hip.decode(q, ks[i], vs[i], out, lse, None, scale=1.0 / math.sqrt(d),
                        num_splits=splits, workspace=ws)

    calls()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        calls()  # warm on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            calls()
    graph.replay()
    torch.cuda.synchronize()
    us = replay_median_us(torch, graph, replays, nsets)
    nbytes = 2 * b * hkv * sk * d * 2 + b * hq * sq * d * 2 * 2 + b * hq * sq * 4
    return dict(workload=f"B={b} Hq={hq} Hkv={hkv} Sq={sq} Sk={sk} D={d} fp16 non-causal",
                num_splits=splits, us_per_call=us, us_per_token=us / sq,
                batch_tokens_per_s=b * sq / (us * 1e-6), algorithmic_bytes=nbytes,
                hbm_gbps=nbytes / (us * 1e-6) / 1e9, hbm_frac=nbytes / (us * 1e-6) / PEAK_HBM,
                timing="HIP graph replays of 32 back-to-back calls over 32 K/V sets (537 MB); "
                       f"median of {REPLAY_BATCHES} batches of {replays} replays")


def bench_config5(torch, _hip, steps=64, seed=500):
    """cache [8, 8, 32768, 64] fp16 with per-sequence
    lengths U[4096, 28000] (seeded); each of `steps` steps appends n in
    [1, 16] tokens per sequence at its own position (append kernel, device
    int64 starts) and decodes Hq=32 query heads x n rows per sequence over its
    visible prefix (split-KV decode with device int32 lengths, splits planned
    from the host-side lengths by kf_decode_num_splits_ragged). All inputs of
    the 64 steps are staged on the GPU first; the 64 (append, decode) pairs are
    captured in one HIP graph, and the median of several replays, each timed
    between two events, is the figure. Unused capacity
    holds NaN, as in the parity test. The same 64 steps are also timed through
    the fused entry (kf_attn_append_decode: the decode launch stores the new
    tokens, no append launch) and its outputs checked against the two-launch
    path's. Bytes per step: append
    2 (K, V) x 2 (read + write) x B Hkv n D x 2; decode K + V of every visible
    prefix + Q + O + LSE."""
    b, hkv, cap, d, hq = 8, 8, 32768, 64, 32
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(4096, 28001, (b,), generator=g).tolist()
    ns = [int(torch.randint(1, 17, (1,), generator=g)) for _ in range(steps)]
    kc = torch.full((b, hkv, cap, d), float("nan"), dtype=torch.float16, device="cuda")
    vc = torch.full_like(kc, float("nan"))
    for i, n in enumerate(lengths):
        kc[i, :, :n] = seeded(torch, (hkv, n, d), 510 + i, torch.float16)
        vc[i, :, :n] = seeded(torch, (hkv, n, d), 520 + i, torch.float16)
    plan = []
    cur = list(lengths)
    app_bytes = dec_bytes = 0
    for t, n in enumerate(ns):
        starts = torch.tensor(cur, dtype=torch.int64, device="cuda")
        cur = [x + n for x in cur]
        seqlens = torch.tensor(cur, dtype=torch.int32, device="cuda")
        maxlen = max(cur)
        nk = seeded(torch, (b, hkv, n, d), 600 + t, torch.float16)
        nv = seeded(torch, (b, hkv, n, d), 700 + t, torch.float16)
        q = seeded(torch, (b, hq, n, d), 800 + t, torch.float16)
        out = torch.empty_like(q)
        splits = _hip.decode_num_splits_ragged(b, hq, hkv, n, cur, d)
        ws = torch.empty(max(256, _hip.decode_workspace_bytes(b, hq, hkv, n, d, splits)),
                         dtype=torch.uint8, device="cuda")
        # Fused append + decode: splits over the old keys plus one for the
        # new tokens, positions = the old lengths.
        old = [x - n for x in cur]
        fsplits = _hip.decode_num_splits_ragged(b, hq, hkv, n, old, d)
        fws = torch.empty(_hip.decode_workspace_bytes(b, hq, hkv, n, d, fsplits + 1),
                          dtype=torch.uint8, device="cuda")
        fused = (torch.tensor(old, dtype=torch.int32, device="cuda"), max(old), fsplits, fws,
                 torch.empty_like(q))
        plan.append((nk, nv, starts, seqlens, maxlen, q, out, splits, ws, fused))
        app_bytes += 2 * 2 * b * hkv * n * d * 2
        dec_bytes += 2 * hkv * d * 2 * sum(cur) + 2 * b * hq * n * d * 2 + b * hq * n * 4
    scale = 1.0 / math.sqrt(d)

    def append(i):
        nk, nv, starts = plan[i][0], plan[i][1], plan[i][2]
        _hip.kv_append(kc, vc, nk, nv, start_dev=starts, max_start=plan[i][4] - nk.shape[2])

    def decode(i):
        _, _, _, seqlens, maxlen, q, out, splits, ws, _ = plan[i]
        _hip.decode(q, kc[:, :, :maxlen], vc[:, :, :maxlen], out, None, seqlens, scale=scale,
                    num_splits=splits, workspace=ws)

    def fused_step(i):
        nk, nv, q = plan[i][0], plan[i][1], plan[i][5]
        prev, maxprev, fsplits, fws, fout = plan[i][9]
        _hip.append_decode(q, kc, vc, nk, nv, fout, None, prev, past_length=0,
                           max_length=maxprev, scale=scale, num_splits=fsplits, workspace=fws)

    def timed(fn):
        # Captured into a HIP graph so the figure is GPU time, not the
        # host's launch rate; replayed once to warm, then timed.
        fn()
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            fn()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        # Replays rewrite the same tokens at the same cache positions, so
        # every replay does the same work.
        return replay_median_us(torch, graph, 1, 1)

    both = timed(lambda: [f(i) for i in range(steps) for f in (append, decode)])
    app = timed(lambda: [append(i) for i in range(steps)])
    dec = timed(lambda: [decode(i) for i in range(steps)])
    fused = timed(lambda: [fused_step(i) for i in range(steps)])
    if not all(bool(torch.isfinite(p[6]).all()) for p in plan):
        raise RuntimeError("config 5: non-finite decode output")
    # The fused outputs must agree with the two-launch path's (fp16 O,
    # atol = rtol = 2e-3; the split partitions differ).
    for p in plan:
        if not torch.allclose(p[9][4].float(), p[6].float(), atol=2e-3, rtol=2e-3):
            raise RuntimeError("config 5: fused append + decode differs from append, decode")
    return {"workload": "BASELINE config 5: cache [8,8,32768,64] fp16, lengths U[4096,28000], "
                        f"{steps} steps of append n in [1,16] + ragged decode Hq=32",
            "steps": steps, "tokens_appended": sum(ns), "us_total": both,
            "us_per_step": both / steps,
            "append": {"us_per_step": app / steps, "bytes": app_bytes,
                       "hbm_gbps": app_bytes / (app * 1e-6) / 1e9,
                       "hbm_frac": app_bytes / (app * 1e-6) / PEAK_HBM},
            "decode": {"us_per_step": dec / steps, "bytes": dec_bytes,
                       "hbm_gbps": dec_bytes / (dec * 1e-6) / 1e9,
                       "hbm_frac": dec_bytes / (dec * 1e-6) / PEAK_HBM,
                       "us_per_token": dec / sum(ns)},
            "fused_append_decode": {
                "us_per_step": fused / steps, "bytes": app_bytes // 2 + dec_bytes,
                "hbm_gbps": (app_bytes // 2 + dec_bytes) / (fused * 1e-6) / 1e9,
                "hbm_frac": (app_bytes // 2 + dec_bytes) / (fused * 1e-6) / PEAK_HBM,
                "note": "kf_attn_append_decode: new tokens read once from their buffer, "
                        "written once to the cache; no append launch"},
            "timing": "64 staged steps captured in one HIP graph; the median of "
                      f"{REPLAY_BATCHES} replays, each between two HIP events (after a warm replay)"}


def bench_forward_only(torch, _hip, cfg, causal, reps=50):
    """Forward (O + LSE) alone, `reps` back-to-back launches between two events."""
    b, hq, hkv, s, d = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["S"], cfg["D"]
    q = seeded(torch, (b, hq, s, d), 101, torch.float16)
    k = seeded(torch, (b, hkv, s, d), 102, torch.float16)
    v = seeded(torch, (b, hkv, s, d), 103, torch.float16)
    out = torch.empty_like(q)
    lse = torch.empty((b, hq, s), device=q.device, dtype=torch.float32)
    fn = lambda: _hip.fwd(q, k, v, out, lse, causal=causal, scale=1.0 / math.sqrt(d))
    fn()
    torch.cuda.synchronize()
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    z.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(z) * 1e3 / reps
    f = fwd_flops(b, hq, s, d) if causal else 4.0 * d * b * hq * s * s
    return {"us_per_call": us, "tflops": f / (us * 1e-6) / 1e12,
            "frac": f / (us * 1e-6) / PEAK_MFMA_F16}


def side_configs(torch, _hip, steps):
    """The other BASELINE configurations, each timed on the GPU."""
    res = {}
    c1 = dict(B=2, Hq=8, Hkv=2, S=512, D=64)
    res["config1_forward"] = dict(
        workload="BASELINE config 1 on the GPU: causal GQA forward B=2 Hq=8 Hkv=2 S=512 D=64 fp16",
        **bench_forward_only(torch, _hip, c1, True))
    res["config2_decode_sweep"] = {}
    for sk in (2048, 4096, 8192, 16384):
        r = bench_decode(torch, _hip, torch.float16, sk)
        res["config2_decode_sweep"][str(sk)] = {k: r[k] for k in
                                                ("us_per_call", "hbm_gbps", "hbm_frac", "num_splits")}
    ms, _, _, per, work, flops, _ = bench_train(torch, _hip, torch.bfloat16, steps, steps // 2)
    res["config3_bf16"] = {"ms_per_step": ms, "tflops": flops / (ms * 1e-3) / 1e12,
                           "frac": flops / (ms * 1e-3) / PEAK_MFMA_F16}
    for dd in (72, 96):
        c4 = dict(B=4, Hq=12, Hkv=12, S=2048, D=dd)
        ms, _, _, per, work, flops, _ = bench_train(torch, _hip, torch.float16, steps, steps // 2, c4,
                                                 causal=False, qkv_scale=1.0)
        res[f"config4_d{dd}"] = {
            "workload": f"BASELINE config 4: non-causal MHA fwd+bwd B=4 H=12 S=2048 D={dd} fp16",
            "ms_per_step": ms, "tflops": flops / (ms * 1e-3) / 1e12,
            "frac": flops / (ms * 1e-3) / PEAK_MFMA_F16,
            "flop_convention": "unpadded D: fwd 4 B H S^2 D, fwd+bwd 3.5x"}
    res["config5_append_decode"] = bench_config5(torch, _hip)
    res["torch_sdpa_same_gpu"] = bench_sdpa_comparison(torch)
    return res


def bench_sdpa_comparison(torch, steps=20, warmup=5):
    """PyTorch's own GPU SDPA (the reference's fallback path, attention.py:126)
    against the HIP kernels on the same MI355X, both through the public
    ``attention`` API with identical synthetic inputs and HIP-event timing
    over back-to-back calls: config 3 fwd+bwd, config 1 forward, config 2
    decode at Sk=16384."""
    import kotflash_amd as kf

    def timed(fn):
        prewarm(torch, fn, PREWARM_MS)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    cases = (
        ("config3_fwd_bwd_us", CFG3, True, True, 0.5),
        ("config1_fwd_us", dict(B=2, Hq=8, Hkv=2, S=512, D=64), True, False, 1.0),
        ("config2_decode_sk16384_us", dict(B=2, Hq=8, Hkv=2, S=1, Sk=16384, D=64), False, False, 1.0),
    )
    out = {"timing": "HIP events over back-to-back public-API calls (host overhead included), "
                     "each after a 200 ms pre-warm"}
    for name, c, causal, bwd, sc in cases:
        sk = c.get("Sk", c["S"])
        q = seeded(torch, (c["B"], c["Hq"], c["S"], c["D"]), 901, torch.float16, sc).requires_grad_(bwd)
        k = seeded(torch, (c["B"], c["Hkv"], sk, c["D"]), 902, torch.float16, sc).requires_grad_(bwd)
        v = seeded(torch, (c["B"], c["Hkv"], sk, c["D"]), 903, torch.float16, sc).requires_grad_(bwd)
        do = seeded(torch, (c["B"], c["Hq"], c["S"], c["D"]), 904, torch.float16)
        row = {}
        for backend in ("hip", "sdpa"):
            def call(backend=backend):
                o = kf.attention(q, k, v, causal=causal, backend=backend)
                if bwd:
                    torch.autograd.grad(o, (q, k, v), do)
            row[backend] = timed(call)
        row["speedup"] = row["sdpa"] / row["hip"]
        out[name] = row
    return out


def cpu_baseline(dtype_name):
    """The reference's SDPA path on host cores (fp32, native GQA, autograd
    backward), timed by the oracle's restatement of it at the config 3 shape."""
    import torch
    from oracle.attention_oracle import sdpa_cpu

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    c = CFG3
    g = torch.Generator().manual_seed(301)
    q = (torch.randn(c["B"], c["Hq"], c["S"], c["D"], generator=g) * 0.5).to(
        getattr(torch, dtype_name)).float().requires_grad_(True)
    k = (torch.randn(c["B"], c["Hkv"], c["S"], c["D"], generator=g) * 0.5).to(
        getattr(torch, dtype_name)).float().requires_grad_(True)
    v = (torch.randn(c["B"], c["Hkv"], c["S"], c["D"], generator=g) * 0.5).to(
        getattr(torch, dtype_name)).float().requires_grad_(True)
    do = torch.randn(c["B"], c["Hq"], c["S"], c["D"], generator=g)

    def step():
        out = sdpa_cpu(q, k, v, causal=True)
        torch.autograd.grad(out, (q, k, v), do)

    step()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    work = 3.5 * fwd_flops(c["B"], c["Hq"], c["S"], c["D"])
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": work / t / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": (f"full config 3 shape (B=2 Hq=16 Hkv=4 S=4096 D=128 causal), fp32 "
                       f"torch SDPA fwd + autograd bwd as the reference's _sdpa path "
                       f"(oracle.sdpa_cpu), median of 5 steps = {t:.3f} s on {cores} "
                       f"threads of {model or 'the host CPU'}")}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n", 1)[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100,
                    help="untimed steps first; ~0.1 s of work lets the GPU clocks settle")
    ap.add_argument("--prewarm-ms", type=float, default=PREWARM_MS,
                    help="untimed steps for this much wall time before the --warmup steps "
                         "(GPU clock ramp); reported in the JSON line")
    ap.add_argument("--dtype", choices=("float16", "bfloat16"), default="float16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-side", action="store_true",
                    help="skip the other BASELINE configurations (1, 2 sweep, 3 bf16, 4, 5)")
    ap.add_argument("--pmc-sample", action="store_true",
                    help="run two config 3 steps plus a calibration fill/copy for rocprofv3 "
                         "--pmc and exit (prints no bench line)")
    ap.add_argument("--only-config5", action="store_true",
                    help="run only the config 5 append/decode loops (two-launch and fused) for "
                         "a kernel trace and exit (prints no bench line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path shards over independent (batch, kv_head) groups with no exchange; "
              "one GPU runs one shard's shape)", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import torch

    import kotflash_amd as kf
    from kotflash_amd import _hip

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    dtype = getattr(torch, args.dtype)
    _hip.lib()
    log(f"device: {torch.cuda.get_device_properties(0).gcnArchName}")
    if args.pmc_sample:
        log(json.dumps(pmc_sample(torch, _hip, dtype)))
        return 0
    if args.only_config5:
        log(json.dumps(bench_config5(torch, _hip)))
        return 0

    ms, wall_ms, dkdv_live, per, work, step_flops, prewarm_steps = bench_train(
        torch, _hip, dtype, args.steps, args.warmup, prewarm_ms=args.prewarm_ms)
    log(f"train step: {ms:.4f} ms (GPU events), {wall_ms:.4f} ms (wall); dkdv live "
        f"{dkdv_live:.4f} ms; isolated per kernel {per}")
    api_ms = bench_api(torch, kf, dtype, max(20, args.steps // 5), 5, args.prewarm_ms)
    log(f"public API step: {api_ms:.4f} ms")
    kernels = {}
    for n, t in per.items():
        kernels[n] = {"ms": t, "tflops": work[n] / (t * 1e-3) / 1e12 if work[n] else None,
                      "frac": work[n] / (t * 1e-3) / PEAK_MFMA_F16 if work[n] else None}
    dom = "bwd_dkdv"
    dom_t = dkdv_live * 1e-3
    roofline = {"kernel": "dkdv_kernel (dK/dV, key-stationary backward)", "bound": "mfma",
                "achieved": work[dom] / dom_t / 1e12, "peak": PEAK_MFMA_F16 / 1e12,
                "unit": "TFLOP/s", "frac": work[dom] / dom_t / PEAK_MFMA_F16,
                "traffic": DKDV_TRAFFIC_BYTES, "work_per_launch": work[dom],
                "avg_launch_ms": dkdv_live,
                "timing": "HIP events around each dK/dV launch on its stream, in a second pass of "
                          "--steps identical steps right after the timed ones (the events add about "
                          "6 us to a step, so the timed steps carry none)"}
    decode = None if args.no_decode else bench_decode(torch, _hip, torch.float16, CFG2["Sk"])
    if decode:
        log(f"decode: {decode}")
    side = None if args.no_side else side_configs(torch, _hip, max(20, args.steps // 4))
    if side:
        log(f"side configs: {json.dumps(side)}")
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.dtype)
    value = step_flops / (ms * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm": {"ms": args.prewarm_ms, "steps": prewarm_steps,
                    "why": "untimed steps before the --warmup steps while the GPU clocks ramp "
                           "(~30 ms of load from idle)"},
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.dtype == "float16" else "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 q/k/v, N(0,1) dO)",
        "config": {"workload": "BASELINE config 3: causal GQA fwd+bwd B=2 Hq=16 Hkv=4 "
                               "Sq=Sk=4096 D=128", "global_batch": CFG3["B"], "seq_len": CFG3["S"],
                   "parallelism": "single GPU"},
        "frac_of_peak": value * 1e12 / PEAK_MFMA_F16,
        "wall_ms_per_step": wall_ms,
        "api_ms_per_step": api_ms,
        "kernels": kernels,
        "roofline": roofline,
        "decode": decode,
        "configs": side,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
