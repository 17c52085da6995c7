"""Generate tests/golden/attention_cases.npz.

The reference repository holds no stored vectors (its tests compare against
torch SDPA at test time), so the fixtures here are computed from the
mathematical definition, independently of the oracle's blockwise algorithm:
dense float64 torch on CPU with softmax(scale Q K^T + mask) V, torch.logsumexp
for LSE and torch.autograd for the gradients (K/V repeat_interleave'd to Hq, so
autograd sums each GQA group). Inputs are drawn from seeded generators and
rounded to float16 first; the stored inputs are the float16 values.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "attention_cases.npz"

# name: (B, Hq, Hkv, Sq, Sk, D, causal, seed)
ATTN_CASES = {
    "gqa_causal_unequal": (1, 4, 2, 37, 53, 16, True, 101),
    "mqa_causal_q_longer": (2, 2, 1, 45, 30, 32, True, 102),
    "mha_noncausal_d72": (1, 2, 2, 20, 70, 72, False, 103),
    "gqa_causal_d96": (1, 4, 1, 33, 33, 96, True, 104),
    "gqa_noncausal_d128": (1, 4, 2, 40, 97, 128, False, 105),
    "cfg1_shape_small": (1, 4, 1, 64, 64, 64, True, 106),
}
# Ragged decode: per-batch visible lengths into a cache of capacity 160.
RAGGED = dict(B=3, Hq=4, Hkv=2, Sq=2, cap=160, D=32, lengths=(17, 160, 75), seed=107)
# Append: cache [2, 2, 24, 8], three new tokens at per-sequence starts.
APPEND = dict(B=2, H=2, cap=24, D=8, n=3, starts=(0, 20), seed=108)


def dense_reference(q, k, v, causal, scale):
    group = q.shape[1] // k.shape[1]
    ke = k.repeat_interleave(group, dim=1)
    ve = v.repeat_interleave(group, dim=1)
    s = torch.matmul(q, ke.transpose(-2, -1)) * scale
    if causal:
        i = torch.arange(q.shape[2])[:, None]
        j = torch.arange(k.shape[2])[None, :]
        s = s.masked_fill(j > i, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    return torch.matmul(torch.softmax(s, dim=-1), ve), lse


def main() -> None:
    data = {}
    for name, (b, hq, hkv, sq, sk, d, causal, seed) in ATTN_CASES.items():
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(b, hq, sq, d, generator=g).half()
        k = torch.randn(b, hkv, sk, d, generator=g).half()
        v = torch.randn(b, hkv, sk, d, generator=g).half()
        do = torch.randn(b, hq, sq, d, generator=g).half()
        scale = 1.0 / math.sqrt(d)
        q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
        out, lse = dense_reference(q64, k64, v64, causal, scale)
        dq, dk, dv = torch.autograd.grad(out, (q64, k64, v64), do.double())
        for key, val in (("q", q), ("k", k), ("v", v), ("do", do)):
            data[f"{name}/{key}"] = val.numpy()
        # Expected values are stored in float32 (relative precision 6e-8).
        data[f"{name}/o"] = out.detach().float().numpy()
        data[f"{name}/lse"] = lse.detach().float().numpy()
        data[f"{name}/dq"] = dq.float().numpy()
        data[f"{name}/dk"] = dk.float().numpy()
        data[f"{name}/dv"] = dv.float().numpy()
        data[f"{name}/meta"] = np.array([b, hq, hkv, sq, sk, d, int(causal)], dtype=np.int64)

    r = RAGGED
    g = torch.Generator().manual_seed(r["seed"])
    q = torch.randn(r["B"], r["Hq"], r["Sq"], r["D"], generator=g).half()
    kc = torch.randn(r["B"], r["Hkv"], r["cap"], r["D"], generator=g).half()
    vc = torch.randn(r["B"], r["Hkv"], r["cap"], r["D"], generator=g).half()
    outs, lses = [], []
    for b, n in enumerate(r["lengths"]):
        o, l_ = dense_reference(q[b:b + 1].double(), kc[b:b + 1, :, :n].double(),
                                vc[b:b + 1, :, :n].double(), False, 1.0 / math.sqrt(r["D"]))
        outs.append(o)
        lses.append(l_)
    data["ragged/q"] = q.numpy()
    data["ragged/k_cache"] = kc.numpy()
    data["ragged/v_cache"] = vc.numpy()
    data["ragged/lengths"] = np.array(r["lengths"], dtype=np.int64)
    data["ragged/o"] = torch.cat(outs).float().numpy()
    data["ragged/lse"] = torch.cat(lses).float().numpy()

    a = APPEND
    g = torch.Generator().manual_seed(a["seed"])
    kc = torch.randn(a["B"], a["H"], a["cap"], a["D"], generator=g).half()
    vc = torch.randn(a["B"], a["H"], a["cap"], a["D"], generator=g).half()
    nk = torch.randn(a["B"], a["H"], a["n"], a["D"], generator=g).half()
    nv = torch.randn(a["B"], a["H"], a["n"], a["D"], generator=g).half()
    ek, ev = kc.clone(), vc.clone()
    for b, s in enumerate(a["starts"]):
        ek[b, :, s:s + a["n"]] = nk[b]
        ev[b, :, s:s + a["n"]] = nv[b]
    data["append/k_cache"] = kc.numpy()
    data["append/v_cache"] = vc.numpy()
    data["append/new_k"] = nk.numpy()
    data["append/new_v"] = nv.numpy()
    data["append/starts"] = np.array(a["starts"], dtype=np.int64)
    data["append/k_expected"] = ek.numpy()
    data["append/v_expected"] = ev.numpy()

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
