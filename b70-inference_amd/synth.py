"""Seeded synthetic EXL3 tensors for the benchmark workloads and the parity tests.

Everything is generated on the CPU from torch.Generator seeds, so the HIP path and the CPU oracle see identical bytes:
  trellis  uniform random int16 over the full range
  suh      random +-1 (fp16)
  svh      random +-1 times the fp16 scale fp16(1 / sqrt(k_in)), which keeps layer outputs O(1) (with unit scales
           the down projection of a 5120-wide MLP would exceed the fp16 range)
  x        N(0, 1) fp16
"""
from __future__ import annotations

import math

import numpy as np
import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(int(seed))


def trellis(k: int, n: int, K: int, g: torch.Generator) -> torch.Tensor:
    return torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g)


def signs(n: int, g: torch.Generator, scale: float = 1.0) -> torch.Tensor:
    s = torch.randint(0, 2, (n,), generator=g).float() * 2 - 1
    return (s * torch.tensor(scale, dtype=torch.float16).float()).half()


def linear(k: int, n: int, K: int, seed: int):
    """(trellis int16 [k/16, n/16, 16K], suh fp16 [k], svh fp16 [n])"""
    g = gen(seed)
    tr = trellis(k, n, K, g)
    suh = signs(k, g)
    svh = signs(n, g, 1.0 / math.sqrt(k))
    return tr, suh, svh


def mixed_linear(k: int, n: int, seed: int, Ks=(1, 2), probs=(0.38, 0.62)):
    """Per-tile K: (words uint32-as-int32 [total], kmap uint8 [tk*tn], woff int32 [tk*tn + 1], suh, svh).
    Tile i (row-major over [k/16, n/16]) holds 8*kmap[i] words at woff[i]."""
    g = gen(seed)
    tk, tn = k // 16, n // 16
    u = torch.rand(tk * tn, generator=g)
    edges = torch.tensor(np.cumsum(probs)[:-1], dtype=torch.float32)
    kmap = torch.tensor(Ks, dtype=torch.uint8)[torch.bucketize(u, edges, right=True)]
    woff = torch.zeros(tk * tn + 1, dtype=torch.int64)
    woff[1:] = torch.cumsum(kmap.to(torch.int64) * 8, 0)
    total = int(woff[-1])
    words = torch.randint(-(2 ** 31), 2 ** 31, (total,), dtype=torch.int64, generator=g).to(torch.int32)
    suh = signs(k, g)
    svh = signs(n, g, 1.0 / math.sqrt(k))
    return words, kmap, woff.to(torch.int32), suh, svh


def activations(m: int, k: int, seed: int) -> torch.Tensor:
    return torch.randn(m, k, generator=gen(seed)).half()
