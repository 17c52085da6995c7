"""CPU oracle for the kotflash_amd attention hot path -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline); the
product path (kotflash_amd) never calls it.

It restates, in float64 numpy, the reference algorithms the HIP kernels
implement, each function citing the reference lines it follows
(paths relative to the reference repository root):

  forward_blockwise   kotflash/kernels/triton_forward.py:20-165
  split_kv_partials   kotflash/kernels/triton_forward.py:169-266
  split_kv_merge      kotflash/kernels/triton_forward.py:269-349
  split_kv_plan       kotflash/_planning.py:25-34
  backward_blockwise  kotflash/attention.py:138-201
  kv_append           kotflash/csrc/kv_append_cuda.cu:12-40 (+ per-sequence start)
  sdpa_cpu            kotflash/attention.py:48-61, 120-135 (torch CPU SDPA)

How each is pinned (tests/test_oracle.py), independently of this file:
  * golden fixtures from tests/golden/make_golden.py (dense closed-form
    softmax / logsumexp / autograd in float64 torch -- a different algorithm);
  * closed forms: q = 0 gives LSE = ln(#visible keys) and O = mean of the
    visible V rows; causal row 0 gives O = V[0]; constant V gives O = V;
  * invariants: split + merge equals the unsplit forward for any split count,
    an empty split has weight 0, the plan partitions [0, Sk);
  * backward against central finite differences of the float64 forward and
    against torch autograd;
  * append against slice assignment (bit-exact) and untouched sentinels;
  * planted mistakes (causal j < i, missing scale, untransposed V) fail them.
No function is left "parity unpinned".

The reference kernels round P (and dS) to the input dtype before their second
product; ``p_dtype`` reproduces that rounding when given.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

NEG_INF = -np.inf


def _as64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def _kv_head(h: int, hq: int, hkv: int) -> int:
    # GQA map: contiguous groups (triton_forward.py:33, triton_backward.py:137).
    return h // (hq // hkv)


def forward_blockwise(q, k, v, *, causal: bool, scale: float, block_m: int = 64,
                      block_n: int = 32, p_dtype=None) -> Tuple[np.ndarray, np.ndarray]:
    """Online-softmax forward (triton_forward.py:20-165).

    For every (batch, q_head, q tile) the running max m, denominator l and
    accumulator acc are updated tile by tile over keys; scores are scaled then
    masked to -inf where j >= Sk or (causal and j > i) (:104-121); causal
    programs stop at key tile cdiv(min(Sk, Sq, (tile+1) BM), BN) (:69-76);
    O = acc / l (:139-158) and LSE = m + ln(l) (:160-165). Returns (O, LSE)
    in float64; O has q's shape, LSE is [B, Hq, Sq].
    """
    q, k, v = _as64(q), _as64(k), _as64(v)
    bsz, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    out = np.zeros((bsz, hq, sq, d))
    lse = np.zeros((bsz, hq, sq))
    for b in range(bsz):
        for h in range(hq):
            kh = _kv_head(h, hq, hkv)
            for m0 in range(0, sq, block_m):
                rows = np.arange(m0, min(m0 + block_m, sq))
                qt = q[b, h, rows]
                m_i = np.full(len(rows), NEG_INF)
                l_i = np.zeros(len(rows))
                acc = np.zeros((len(rows), d))
                if causal:
                    end = math.ceil(min(sk, sq, m0 + block_m) / block_n)
                else:
                    end = math.ceil(sk / block_n)
                for t in range(end):
                    cols = np.arange(t * block_n, (t + 1) * block_n)
                    valid = cols[None, :] < sk
                    if causal:
                        valid = valid & (cols[None, :] <= rows[:, None])
                    kc = np.where(cols[:, None] < sk, k[b, kh, np.minimum(cols, sk - 1)], 0.0)
                    vc = np.where(cols[:, None] < sk, v[b, kh, np.minimum(cols, sk - 1)], 0.0)
                    s = np.where(valid, (qt @ kc.T) * scale, NEG_INF)
                    m_new = np.maximum(m_i, s.max(axis=1))
                    safe = np.where(np.isneginf(m_new), 0.0, m_new)
                    alpha = np.where(np.isneginf(m_i), 0.0, np.exp(m_i - safe))
                    p = np.where(valid, np.exp(s - safe[:, None]), 0.0)
                    l_i = l_i * alpha + p.sum(axis=1)
                    pc = p if p_dtype is None else p.astype(p_dtype).astype(np.float64)
                    acc = acc * alpha[:, None] + pc @ vc
                    m_i = m_new
                with np.errstate(divide="ignore", invalid="ignore"):
                    out[b, h, rows] = np.where(l_i[:, None] > 0, acc / l_i[:, None], 0.0)
                    lse[b, h, rows] = np.where(l_i > 0, m_i + np.log(l_i), NEG_INF)
    return out, lse


def split_kv_plan(sq: int, sk: int, d: int, *, causal: bool):
    """(num_splits, chunk_n, blocks_per_split) of the reference plan, or None
    (_planning.py:25-34)."""
    if causal or sq > 16 or sk < 1024 or d > 64:
        return None
    splits = min(16, -(-sk // 128))
    chunk = -(-sk // splits)
    return splits, chunk, -(-chunk // 64)


def split_kv_partials(q, k, v, *, scale: float, num_splits: int, chunk_n: int,
                      seqlens=None) -> Tuple[np.ndarray, np.ndarray]:
    """Per-split normalized partial O and partial LSE (triton_forward.py
    :169-266): split s covers keys [s chunk_n, min((s+1) chunk_n, L_b)); a
    split with l = 0 gets O_s = 0 and LSE_s = -inf (:240-246). ``seqlens``
    (per-batch visible key counts) extends the reference for ragged caches.
    Returns part_o [S, B, Hq, Sq, D], part_lse [S, B, Hq, Sq]."""
    q, k, v = _as64(q), _as64(k), _as64(v)
    bsz, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    part_o = np.zeros((num_splits, bsz, hq, sq, d))
    part_lse = np.full((num_splits, bsz, hq, sq), NEG_INF)
    for s in range(num_splits):
        for b in range(bsz):
            length = sk if seqlens is None else int(seqlens[b])
            k0, k1 = s * chunk_n, min((s + 1) * chunk_n, length)
            if k1 <= k0:
                continue
            for h in range(hq):
                kh = _kv_head(h, hq, hkv)
                sc = (q[b, h] @ k[b, kh, k0:k1].T) * scale
                m = sc.max(axis=1)
                p = np.exp(sc - m[:, None])
                l_i = p.sum(axis=1)
                part_o[s, b, h] = (p @ v[b, kh, k0:k1]) / l_i[:, None]
                part_lse[s, b, h] = m + np.log(l_i)
    return part_o, part_lse


def split_kv_merge(part_o, part_lse) -> Tuple[np.ndarray, np.ndarray]:
    """LSE-weighted merge (triton_forward.py:269-349): w_s = exp(LSE_s - max)
    / sum_t exp(LSE_t - max), O = sum_s w_s O_s, LSE = max + ln(sum) or -inf
    when every split is empty."""
    part_o, part_lse = _as64(part_o), _as64(part_lse)
    row_max = part_lse.max(axis=0)
    safe_max = np.where(np.isneginf(row_max), 0.0, row_max)
    w = np.exp(part_lse - safe_max[None])
    denom = w.sum(axis=0)
    safe_den = np.where(denom > 0, denom, 1.0)
    out = (w[..., None] * part_o).sum(axis=0) / safe_den[..., None]
    with np.errstate(divide="ignore"):
        lse = np.where(denom > 0, row_max + np.log(np.where(denom > 0, denom, 1.0)), NEG_INF)
    return out, lse


def backward_blockwise(q, k, v, out, lse, dout, *, causal: bool, scale: float,
                       q_block: int = 64, kv_block: int = 128, p_dtype=None):
    """Recompute-based backward (kotflash/attention.py:138-201, the same math
    as the Triton kernels triton_backward.py:17-195): delta = rowsum(O dO)
    from the given (stored) O; per tile P = exp(scale S - LSE) masked,
    dP = dO V^T, dS = P (dP - delta), dQ += scale dS K,
    dK += scale dS^T Q, dV += P^T dO, with dK/dV summed over each GQA group.
    ``p_dtype`` rounds P and dS before the products like the kernels
    (triton_backward.py:85, :183-184). Returns float64 (dq, dk, dv)."""
    q, k, v, out, dout = (_as64(x) for x in (q, k, v, out, dout))
    lse = _as64(lse)
    bsz, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    rnd = (lambda x: x) if p_dtype is None else (lambda x: x.astype(p_dtype).astype(np.float64))
    for b in range(bsz):
        for h in range(hq):
            kh = _kv_head(h, hq, hkv)
            for q0 in range(0, sq, q_block):
                rows = np.arange(q0, min(q0 + q_block, sq))
                qb, gb = q[b, h, rows], dout[b, h, rows]
                delta = (out[b, h, rows] * gb).sum(axis=1)
                for k0 in range(0, sk, kv_block):
                    cols = np.arange(k0, min(k0 + kv_block, sk))
                    kb, vb = k[b, kh, cols], v[b, kh, cols]
                    s = (qb @ kb.T) * scale
                    if causal:
                        s = np.where(cols[None, :] > rows[:, None], NEG_INF, s)
                    with np.errstate(over="ignore", invalid="ignore"):
                        p = np.exp(s - lse[b, h, rows][:, None])
                    p = np.nan_to_num(p, nan=0.0, posinf=0.0, neginf=0.0)
                    ds = p * (gb @ vb.T - delta[:, None])
                    dq[b, h, rows] += (rnd(ds) @ kb) * scale
                    dk[b, kh, cols] += (rnd(ds).T @ qb) * scale
                    dv[b, kh, cols] += rnd(p).T @ gb
    return dq, dk, dv


def kv_append(k_cache, v_cache, new_k, new_v, start) -> None:
    """In-place cache append (kv_append_cuda.cu:12-40): every element of new
    [B, H, S, D] is copied to cache[b, h, start + t, d], walking the same
    linear index decomposition d, t, h, b as the reference kernel (:29-32).
    ``start`` may be a scalar or a per-batch sequence of positions (the
    per-sequence extension). Works on any numpy dtype, bit-exact."""
    bsz, heads, seq, dim = new_k.shape
    starts = [int(start)] * bsz if np.isscalar(start) else [int(s) for s in start]
    total = bsz * heads * seq * dim
    for linear in range(total):
        dd = linear % dim
        t = (linear // dim) % seq
        h = (linear // (dim * seq)) % heads
        b = linear // (dim * seq * heads)
        k_cache[b, h, starts[b] + t, dd] = new_k[b, h, t, dd]
        v_cache[b, h, starts[b] + t, dd] = new_v[b, h, t, dd]


def sdpa_cpu(q, k, v, *, causal: bool, scale: Optional[float] = None):
    """The reference's SDPA path on CPU torch tensors (kotflash/attention.py
    :48-61, :120-135): native-GQA ``scaled_dot_product_attention``, with
    ``scale`` omitted when it equals 1/sqrt(D). This is the reference's only
    implementation that runs on an MI355X host, timed as the CPU baseline."""
    import torch
    import torch.nn.functional as F

    kwargs = {"attn_mask": None, "dropout_p": 0.0, "is_causal": causal}
    if scale is not None and not math.isclose(scale, 1.0 / math.sqrt(q.shape[-1]),
                                              rel_tol=0.0, abs_tol=1e-12):
        kwargs["scale"] = scale
    if q.shape[1] != k.shape[1]:
        return F.scaled_dot_product_attention(q, k, v, enable_gqa=True, **kwargs)
    return F.scaled_dot_product_attention(q, k, v, **kwargs)
