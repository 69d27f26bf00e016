"""Seeded synthetic paged KV for the codec workloads.

Value model: K[token, h, d] = N(0, 1) * s[h, d] with s drawn log-uniform from
[0.1, 10] per channel and layer; V = N(0, 0.5). Both are rounded to bf16
(round-to-nearest-even, torch's cast). Optionally a fraction of the elements is
replaced by outliers of magnitude log-uniform in [1e2, 1e4] with a random sign.
A layer is a vLLM paged cache tensor (2, num_blocks, block_size, kv_heads,
head_dim); request r owns a random, non-contiguous list of block ids.
Every draw comes from torch generators seeded with seed * 1000 + layer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

from . import codebooks as cb


@dataclass(frozen=True)
class Shape:
    layers: int
    kv_heads: int
    head_dim: int
    block_size: int = 16

    @property
    def block_words(self) -> int:
        return self.block_size * self.kv_heads * self.head_dim


LLAMA32_1B = Shape(layers=16, kv_heads=8, head_dim=64)
LLAMA3_8B = Shape(layers=32, kv_heads=8, head_dim=128)
LLAMA3_70B_TP8 = Shape(layers=80, kv_heads=1, head_dim=128)


def _generator(torch, device, seed: int):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_kv_layer(torch, shape: Shape, num_blocks: int, *, seed: int, layer: int, device,
                  outlier_rate: float = 0.0):
    """One paged layer (2, num_blocks, block_size, kv_heads, head_dim) in bf16."""
    g = _generator(torch, device, seed * 1000 + layer)
    dims = (num_blocks, shape.block_size, shape.kv_heads, shape.head_dim)
    lo, hi = math.log(0.1), math.log(10.0)
    scale = torch.exp(torch.rand((shape.kv_heads, shape.head_dim), generator=g, device=device)
                      * (hi - lo) + lo)
    kv = torch.empty((2,) + dims, dtype=torch.bfloat16, device=device)
    kv[0] = (torch.randn(dims, generator=g, device=device) * scale).to(torch.bfloat16)
    kv[1] = (torch.randn(dims, generator=g, device=device) * 0.5).to(torch.bfloat16)
    if outlier_rate > 0:
        flat = kv.view(-1)
        mask = torch.rand(flat.shape, generator=g, device=device) < outlier_rate
        count = int(mask.sum().item())
        mag = torch.exp(torch.rand(count, generator=g, device=device)
                        * (math.log(1e4) - math.log(1e2)) + math.log(1e2))
        sign = torch.where(torch.rand(count, generator=g, device=device) < 0.5, -1.0, 1.0)
        flat[mask] = (mag * sign).to(torch.bfloat16)
    return kv


def random_block_tables(torch, pool_blocks: int, blocks_per_request, *, seed: int):
    """Request r gets the next blocks_per_request[r] ids of one seeded permutation
    of the pool (non-contiguous, random order)."""
    g = _generator(torch, "cpu", seed)
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    tables, at = [], 0
    for count in blocks_per_request:
        if at + count > pool_blocks:
            raise ValueError("pool too small for the requested blocks")
        tables.append(perm[at:at + count])
        at += count
    return tables


def mixed_context_lengths(torch, requests: int, lo: int, hi: int, block_size: int, *, seed: int):
    """Token counts log-uniform over [lo, hi], rounded up to whole blocks."""
    g = _generator(torch, "cpu", seed)
    u = torch.rand(requests, generator=g, dtype=torch.float64)
    tokens = torch.exp(u * (math.log(hi) - math.log(lo)) + math.log(lo))
    return [int(-(-int(math.ceil(t)) // block_size) * block_size) for t in tokens.tolist()]


def exponent_histograms(torch, kv_layer, block_tables):
    """(2, 256) int64 counts of bf16 exponents over every request's blocks of the
    layer, K plane and V plane separately (what the connector's exponent trace
    records, src/unchain_kv/vllm_connector.py:2871-2904)."""
    ids = torch.tensor([b for t in block_tables for b in t], dtype=torch.int64,
                       device=kv_layer.device)
    out = []
    for plane in range(2):
        words = kv_layer[plane].index_select(0, ids).reshape(-1).view(torch.int16).to(torch.int32)
        exps = torch.bitwise_and(torch.bitwise_right_shift(words, 7), 0xFF)
        out.append(torch.bincount(exps, minlength=256))
    return torch.stack(out)


def fit_codebook(torch, kv_layer, block_tables) -> bytes:
    """Per-layer Top-16 codebook fit on the same tensor (K then V)."""
    hist = exponent_histograms(torch, kv_layer, block_tables).cpu().tolist()
    return cb.fit_layer_codebook(hist[0], hist[1])

