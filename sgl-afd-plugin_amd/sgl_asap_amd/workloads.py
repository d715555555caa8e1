"""Seeded synthetic MoE-layer jobs (inputs, routing, expert weights) for benchmarks and tests.

The reference's only input generator is the FFN-rank warm-up
(``python/sgl_asap_plugin/srt/managers/scheduler.py:329-351``: a seeded generator, x ~ randn
bf16, top-k of random scores). The shapes and distributions here are the benchmark
workloads of this path:

* ``tiny``       hidden 256, inter 128, 8 experts (all local), top-2, 64 tokens.
* ``dsv4_rank``  hidden 4096, inter 2048, 256 experts of which rank 0 owns [0, 64), top-8,
                 uniform routing, 16384 tokens, MXFP4 weights.
* ``dsv4_zipf``  the same shape, expert popularity Zipf(1.2) over a seeded permutation of
                 the 256 experts; job sizes log-uniform in [256, 16384].
* ``ernie_fp8``  hidden 4096, inter 1536, 64 experts all local, top-8, Zipf(1.1),
                 FP8-e4m3 weights with 128x128 block scales.

Routing: logits ~ N(0,1) -> softmax -> top-k -> renormalised weights (uniform case); the
skewed cases draw k distinct experts by Gumbel-top-k on log p with p ~ Zipf. Expert weights
~ N(0, 0.02) in fp32 before quantization. Everything comes from one torch.Generator seeded
by ``seed`` on the requested device, in a fixed order.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch


@dataclass(frozen=True)
class MoeShape:
    name: str
    hidden: int
    inter: int
    num_experts: int  # global experts
    num_local: int  # experts of F rank 0: [0, num_local)
    top_k: int
    tokens: int
    fmt: str  # "mxfp4" or "fp8_block"
    zipf: Optional[float] = None  # None = uniform routing

    @property
    def local(self) -> range:
        return range(0, self.num_local)


SHAPES = {
    "tiny": MoeShape("tiny", 256, 128, 8, 8, 2, 64, "mxfp4"),
    "dsv4_rank": MoeShape("dsv4_rank", 4096, 2048, 256, 64, 8, 16384, "mxfp4"),
    "dsv4_zipf": MoeShape("dsv4_zipf", 4096, 2048, 256, 64, 8, 16384, "mxfp4", zipf=1.2),
    "ernie_fp8": MoeShape("ernie_fp8", 4096, 1536, 64, 64, 8, 16384, "fp8_block", zipf=1.1),
}


def generator(device, seed: int = 0) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def tokens(n: int, hidden: int, gen: torch.Generator, device) -> torch.Tensor:
    """x ~ N(0, 1) in bf16."""
    return torch.randn(n, hidden, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)


def route_uniform(n: int, num_experts: int, top_k: int, gen: torch.Generator, device):
    """logits ~ N(0,1) -> softmax -> top-k -> renormalise. -> (ids i32 [n,k], w f32 [n,k])."""
    logits = torch.randn(n, num_experts, generator=gen, device=device, dtype=torch.float32)
    probs = torch.softmax(logits, dim=-1)
    w, ids = torch.topk(probs, top_k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return ids.to(torch.int32), w.to(torch.float32)


def zipf_popularity(num_experts: int, alpha: float, gen: torch.Generator, device) -> torch.Tensor:
    """p[e] proportional to rank(e)^-alpha, ranks assigned by a seeded permutation."""
    ranks = torch.randperm(num_experts, generator=gen, device=device).to(torch.float64) + 1.0
    p = ranks.pow(-alpha)
    return (p / p.sum()).to(torch.float32)


def route_zipf(n: int, num_experts: int, top_k: int, alpha: float, gen: torch.Generator, device):
    """k distinct experts per token by Gumbel-top-k on log p (p ~ Zipf(alpha)); weights are
    the renormalised softmax of N(0,1) logits at the chosen experts."""
    p = zipf_popularity(num_experts, alpha, gen, device)
    u = torch.rand(n, num_experts, generator=gen, device=device, dtype=torch.float32)
    gumbel = -torch.log(-torch.log(u.clamp_min(1e-20)))
    _, ids = torch.topk(p.log()[None, :] + gumbel, top_k, dim=-1)
    logits = torch.randn(n, top_k, generator=gen, device=device, dtype=torch.float32)
    w = torch.softmax(logits, dim=-1)
    return ids.to(torch.int32), w.to(torch.float32)


def expert_weights(num_local: int, hidden: int, inter: int, gen: torch.Generator, device, std: float = 0.02):
    """Logical fp32 weights: w13 [E, 2I, H] = [gate; up], w2 [E, H, I], ~ N(0, std)."""
    w13 = torch.randn(num_local, 2 * inter, hidden, generator=gen, device=device, dtype=torch.float32) * std
    w2 = torch.randn(num_local, hidden, inter, generator=gen, device=device, dtype=torch.float32) * std
    return w13, w2


def job(shape: MoeShape, n: Optional[int] = None, seed: int = 0, device="cpu"):
    """(x, ids, w) of one job of ``shape`` (n tokens, default shape.tokens)."""
    n = shape.tokens if n is None else n
    gen = generator(device, seed)
    x = tokens(n, shape.hidden, gen, device)
    if shape.zipf is None:
        ids, w = route_uniform(n, shape.num_experts, shape.top_k, gen, device)
    else:
        ids, w = route_zipf(n, shape.num_experts, shape.top_k, shape.zipf, gen, device)
    return x, ids, w


def job_sizes(count: int, lo: int = 256, hi: int = 16384, seed: int = 0) -> list:
    """Token counts log-uniform in [lo, hi] (the skewed job stream), host-side."""
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(count, generator=g, dtype=torch.float64)
    return [int(round(math.exp(math.log(lo) + float(v) * (math.log(hi) - math.log(lo))))) for v in u]


def pair_count(ids: torch.Tensor, local: range) -> int:
    """Np: local (token, expert) pairs of a job, counted from the generated ids."""
    return int(((ids >= local.start) & (ids < local.stop)).sum().item())


def flops(shape_hidden: int, inter: int, np_pairs: int) -> int:
    """Algorithmic FLOPs of the expert path: 2*H*2I (gate_up) + 2*I*H (down) per pair."""
    return 6 * shape_hidden * inter * np_pairs
