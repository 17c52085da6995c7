"""Decoder-block training step with each attention backend, on one GPU.

    python -m kotflash_amd.benchmark_decoder_block --batch 2 --seq 4096 --q-heads 16 --kv-heads 4 --head-dim 128

The end-to-end consumer of the forward and backward kernels, with the same
arguments and report fields as the reference's decoder-block benchmark
(benchmarks/benchmark_decoder_block.py:34-260):

- The block is pre-norm: LayerNorm, then Q/K/V projections with grouped KV
  heads, causal attention and the output projection; then LayerNorm and a
  SiLU-gated MLP.
- Parameters and activations are fp32 (AdamW master weights), and Q/K/V are
  cast to the attention dtype (fp16 by default) for every backend.
- Each backend trains its own copy of one initial state. Reported per
  backend: the median step time, tokens per second, the incremental peak of
  allocated memory, and whether the loss and the updated parameters are
  finite.
- Backends are ``sdpa_expanded_kv``, ``sdpa_native_gqa`` and ``hip`` (this
  build's kernels; the reference's ``triton`` slot).
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
from typing import List, Optional

import torch
import torch.nn.functional as F
from torch import nn

from .attention import attention

BACKENDS = ("sdpa_expanded_kv", "sdpa_native_gqa", "hip")


class DecoderBlock(nn.Module):
    """Pre-norm decoder block with GQA/MQA projections and a gated MLP."""

    def __init__(self, q_heads: int, kv_heads: int, head_dim: int, mlp_ratio: int = 4,
                 attention_dtype: torch.dtype = torch.float16):
        super().__init__()
        hidden, kv_width = q_heads * head_dim, kv_heads * head_dim
        self.q_heads, self.kv_heads, self.head_dim = q_heads, kv_heads, head_dim
        self.attention_dtype = attention_dtype
        self.norm1 = nn.LayerNorm(hidden)
        self.q_proj = nn.Linear(hidden, hidden, bias=False)
        self.k_proj = nn.Linear(hidden, kv_width, bias=False)
        self.v_proj = nn.Linear(hidden, kv_width, bias=False)
        self.o_proj = nn.Linear(hidden, hidden, bias=False)
        self.norm2 = nn.LayerNorm(hidden)
        self.gate_proj = nn.Linear(hidden, hidden * mlp_ratio, bias=False)
        self.up_proj = nn.Linear(hidden, hidden * mlp_ratio, bias=False)
        self.down_proj = nn.Linear(hidden * mlp_ratio, hidden, bias=False)

    def _heads(self, t: torch.Tensor, heads: int) -> torch.Tensor:
        b, s, _ = t.shape
        return t.view(b, s, heads, self.head_dim).transpose(1, 2).to(self.attention_dtype)

    def forward(self, x: torch.Tensor, backend: str) -> torch.Tensor:
        b, s, hidden = x.shape
        h = self.norm1(x)
        q = self._heads(self.q_proj(h), self.q_heads)
        k = self._heads(self.k_proj(h), self.kv_heads)
        v = self._heads(self.v_proj(h), self.kv_heads)
        if backend == "hip":
            a = attention(q, k, v, causal=True, backend="hip")
        elif backend == "sdpa_native_gqa":
            a = attention(q, k, v, causal=True, backend="sdpa")
        elif backend == "sdpa_expanded_kv":
            g = self.q_heads // self.kv_heads
            a = F.scaled_dot_product_attention(q, k.repeat_interleave(g, dim=1),
                                               v.repeat_interleave(g, dim=1), is_causal=True)
        else:
            raise ValueError(f"unknown attention backend: {backend}")
        a = a.transpose(1, 2).reshape(b, s, hidden).to(x.dtype)
        x = x + self.o_proj(a)
        h = self.norm2(x)
        return x + self.down_proj(F.silu(self.gate_proj(h)) * self.up_proj(h))


def _train_step(model, opt, x, target, backend):
    opt.zero_grad(set_to_none=True)
    loss = F.mse_loss(model(x, backend), target)
    loss.backward()
    opt.step()
    return loss.detach()


def _run_backend(backend, state, x, target, args, attention_dtype) -> dict:
    model = DecoderBlock(args.q_heads, args.kv_heads, args.head_dim,
                         attention_dtype=attention_dtype).to(x.device)
    model.load_state_dict(state)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
    for _ in range(args.warmup):
        _train_step(model, opt, x, target, backend)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(x.device)
    torch.cuda.reset_peak_memory_stats(x.device)
    marks, loss = [], None
    for _ in range(args.iterations):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        loss = _train_step(model, opt, x, target, backend)
        e1.record()
        marks.append((e0, e1))
    torch.cuda.synchronize()
    ms = statistics.median(a.elapsed_time(z) for a, z in marks)
    loss_value = float(loss.item())
    return {
        "median_step_ms": ms,
        "tokens_per_second": x.shape[0] * x.shape[1] * 1e3 / ms,
        "incremental_peak_allocated_bytes": max(0, torch.cuda.max_memory_allocated(x.device) - base),
        "last_loss": loss_value,
        "loss_finite": math.isfinite(loss_value),
        "parameters_finite_after_update": all(bool(torch.isfinite(p).all()) for p in model.parameters()),
    }


def run(args: argparse.Namespace) -> dict:
    torch.manual_seed(1234)
    device = torch.device("cuda")
    attention_dtype = torch.bfloat16 if args.attention_dtype == "bf16" else torch.float16
    hidden = args.q_heads * args.head_dim
    x = torch.randn(args.batch, args.seq, hidden, device=device)
    target = torch.randn_like(x)
    template = DecoderBlock(args.q_heads, args.kv_heads, args.head_dim)
    state = {k: v.detach().clone() for k, v in template.state_dict().items()}
    props = torch.cuda.get_device_properties(device)
    report = {
        "gpu": torch.cuda.get_device_name(device),
        "arch": getattr(props, "gcnArchName", None),
        "torch": torch.__version__,
        "hip_runtime": getattr(torch.version, "hip", None),
        "shape": {"batch": args.batch, "sequence": args.seq, "q_heads": args.q_heads,
                  "kv_heads": args.kv_heads, "head_dim": args.head_dim, "hidden_size": hidden},
        "model_parameter_dtype": "torch.float32",
        "attention_compute_dtype": str(attention_dtype),
        "optimizer": "AdamW with fp32 master parameters",
        "warmup": args.warmup,
        "iterations": args.iterations,
    }
    backends = list(BACKENDS)
    try:
        ref_model = DecoderBlock(args.q_heads, args.kv_heads, args.head_dim,
                                 attention_dtype=attention_dtype).to(device)
        ref_model.load_state_dict(state)
        with torch.no_grad():
            ref = ref_model(x, "sdpa_expanded_kv")
            got = ref_model(x, "hip")
        report["max_abs_output_error_vs_expanded_sdpa"] = (got - ref).abs().max().item()
        report["hip_output_finite"] = bool(torch.isfinite(got).all())
        del ref_model, ref, got
    except Exception as exc:  # recorded: the hip backend is then skipped
        backends.remove("hip")
        report["hip_forward"] = {"unavailable_or_failed": f"{type(exc).__name__}: {exc}"}
    torch.cuda.empty_cache()
    for backend in backends:
        report[backend] = _run_backend(backend, state, x, target, args, attention_dtype)
    if "hip" in report:
        for base in ("sdpa_expanded_kv", "sdpa_native_gqa"):
            report[f"hip_speedup_vs_{base}"] = (
                report[base]["median_step_ms"] / report["hip"]["median_step_ms"])
    return report


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--batch", type=int, default=2)
    p.add_argument("--seq", type=int, default=512)
    p.add_argument("--q-heads", type=int, default=8)
    p.add_argument("--kv-heads", type=int, default=2)
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--iterations", type=int, default=10)
    p.add_argument("--attention-dtype", choices=("fp16", "bf16"), default="fp16")
    args = p.parse_args(argv)
    if min(args.batch, args.seq, args.q_heads, args.kv_heads, args.head_dim) <= 0:
        p.error("batch, sequence length, head counts and head dimension must be positive")
    if args.q_heads % args.kv_heads:
        p.error("--q-heads must be divisible by --kv-heads")
    if args.warmup < 1 or args.iterations < 3:
        p.error("use at least one warmup and three measured iterations")
    if not torch.cuda.is_available():
        p.error("a GPU is required")
    return args


def main(argv: Optional[List[str]] = None) -> None:
    print(json.dumps(run(parse_args(argv)), indent=2, default=str))


if __name__ == "__main__":
    main()
