"""Seeded synthetic experts shared by the MoE tests and the benchmark checks: the same CPU bytes feed the GPU tables
and the oracle's Proj objects."""
import importlib

import numpy as np
import torch

synth = importlib.import_module("b70-inference_amd.synth")


def make_proj(k, n, K, seed, per_tile=None):
    """Uniform K: (tr, suh, svh). per_tile=(Ks, probs): (words, kmap, woff, suh, svh)."""
    if per_tile is None:
        return synth.linear(k, n, K, seed)
    return synth.mixed_linear(k, n, seed, *per_tile)


def oracle_proj(O, cpu):
    if len(cpu) == 3:
        tr, suh, svh = cpu
        return O.Proj(suh.numpy(), svh.numpy(), trellis=tr.numpy(), K=tr.shape[-1] // 16)
    words, kmap, woff, suh, svh = cpu
    return O.Proj(suh.numpy(), svh.numpy(), words=words.numpy().view(np.uint32), kmap=kmap.numpy(),
                  woff=woff.numpy().astype(np.int64))


def gpu_proj(exl3, cpu, dev):
    if len(cpu) == 3:
        tr, suh, svh = cpu
        return exl3.BC_LinearEXL3(tr.to(dev), suh.to(dev), svh.to(dev), tr.shape[-1] // 16, None, False, True, None)
    return exl3.MixedEXL3(*(t.to(dev) for t in cpu))


def make_experts(exl3, O, E, H, I, Kgu, Kd, seed, per_tile=None, dev="cuda", oracle=True):
    """Returns (ExpertTables on dev, list of oracle (gate, up, down) Proj tuples or None)."""
    gates, ups, downs, orc = [], [], [], []
    for e in range(E):
        cg = make_proj(H, I, Kgu, seed + 10 * e + 0, per_tile)
        cu = make_proj(H, I, Kgu, seed + 10 * e + 1, per_tile)
        cd = make_proj(I, H, Kd, seed + 10 * e + 2, per_tile)
        gates.append(gpu_proj(exl3, cg, dev))
        ups.append(gpu_proj(exl3, cu, dev))
        downs.append(gpu_proj(exl3, cd, dev))
        if oracle:
            orc.append((oracle_proj(O, cg), oracle_proj(O, cu), oracle_proj(O, cd)))
    return exl3.ExpertTables(gates, ups, downs), (orc if oracle else None)


def max_rel(y, r):
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    return float(np.abs(y - r).max() / np.abs(r).max())
