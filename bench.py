#!/usr/bin/env python3
"""Benchmark of the EXL3 quantized-linear + MoE-expert hot path on one MI355X.

One step = one layer call of the headline workload (C3 below) on 4 decode tokens: softmax/top-10 routing from fp32
logits and the grouped MoE layer (gate|up + activation, down, combine) in one library call (moe_forward_logits). Timed as HIP-graph replay of exactly
--steps steps (warmup steps run eagerly first); every step uses a fresh routing and cycles through layer copies so the
expert weights come from HBM, not the 256 MB Infinity Cache. Prints one JSON line.

Workloads (seeded synthetic EXL3 tensors generated on the device; parity is tested separately against the oracle):
  C1  dense linear 4096 -> 4096, K=4, 1 token
  C2  dense MLP 5376 <-> 21504, K=4, GELU-tanh gate, 1 / 2 / 4 tokens
  C3  MoE decode layer H=2048, 512 experts of I=512, K=3, top-10 softmax, SiLU, 1 / 2 / 4 tokens   (headline)
  C4  MoE prefill layer H=5120, 160 experts of I=1536, gate/up K=2 + down K=3, top-8 softmax over logits + Zipf(1.1)
      expert bias, 512 tokens
  C5  MoE layer H=7168, 256 experts of I=2048 + 1 shared, per-tile K in {1, 2} (38/62), top-8, 4 decode + 256
      prefill rows in one call
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "EXL3 MoE layer µs/token + achieved HBM GB/s (% of peak), 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

exl3 = importlib.import_module("b70-inference_amd")


def log(*a):
    print("bench:", *a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------------ weights
def dev_gen(seed):
    return torch.Generator(device="cuda").manual_seed(int(seed))


def dev_linear(k, n, K, g):
    tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
    suh = (torch.randint(0, 2, (k,), device="cuda", generator=g).float() * 2 - 1).half()
    svh = ((torch.randint(0, 2, (n,), device="cuda", generator=g).float() * 2 - 1) *
           float(torch.tensor(1.0 / math.sqrt(k)).half())).half()
    return exl3.BC_LinearEXL3(tr, suh, svh, K, None, False, True, None)


def dev_mixed(k, n, g, Ks=(1, 2), probs=(0.38, 0.62)):
    tk, tn = k // 16, n // 16
    u = torch.rand(tk * tn, device="cuda", generator=g)
    kmap = torch.full((tk * tn,), Ks[-1], dtype=torch.uint8, device="cuda")
    acc = 0.0
    for K, p in zip(Ks[:-1], probs[:-1]):
        kmap[(u >= acc) & (u < acc + p)] = K
        acc += p
    woff = torch.zeros(tk * tn + 1, dtype=torch.int64, device="cuda")
    woff[1:] = torch.cumsum(kmap.to(torch.int64) * 8, 0)
    total = int(woff[-1])
    words = torch.randint(-(2 ** 31), 2 ** 31, (total,), dtype=torch.int64, device="cuda", generator=g).to(torch.int32)
    suh = (torch.randint(0, 2, (k,), device="cuda", generator=g).float() * 2 - 1).half()
    svh = ((torch.randint(0, 2, (n,), device="cuda", generator=g).float() * 2 - 1) *
           float(torch.tensor(1.0 / math.sqrt(k)).half())).half()
    return exl3.MixedEXL3(words, kmap, woff.to(torch.int32), suh, svh)


def dev_packed(E, k, n, K, g):
    """E projections k -> n generated straight into one [E, ...] allocation per tensor kind (uniform strides)."""
    tr = torch.randint(-32768, 32768, (E, k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
    suh = (torch.randint(0, 2, (E, k), device="cuda", generator=g).float() * 2 - 1).half()
    svh = ((torch.randint(0, 2, (E, n), device="cuda", generator=g).float() * 2 - 1) *
           float(torch.tensor(1.0 / math.sqrt(k)).half())).half()
    return [exl3.BC_LinearEXL3(tr[e], suh[e], svh[e], K, None, False, True, None) for e in range(E)]


def dev_experts(E, H, I, Kgu, Kd, seed, mixed=False):
    """Expert tables with random weights: uniform K packed per projection as a model loader lays them out
    (ExpertTables.packed), per-tile K one allocation per projection."""
    g = dev_gen(seed)
    if not mixed:
        return exl3.ExpertTables(dev_packed(E, H, I, Kgu, g), dev_packed(E, H, I, Kgu, g), dev_packed(E, I, H, Kd, g))
    gates, ups, downs = [], [], []
    for _ in range(E):
        gates.append(dev_mixed(H, I, g))
        ups.append(dev_mixed(H, I, g))
        downs.append(dev_mixed(I, H, g))
    return exl3.ExpertTables(gates, ups, downs)


def proj_bytes(p):
    b = p.trellis.numel() * p.trellis.element_size() + 2 * (p.in_features + p.out_features)
    if isinstance(p, exl3.MixedEXL3):
        b += p.kmap.numel() + 4 * p.woff.numel()
    return b


# ------------------------------------------------------------------------------------------------ timing
def graph_time(fns, reps=1, wall=False):
    """Capture fns (in order) into one HIP graph, replay `reps` times; returns (us per fn call, wall seconds)."""
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    g.replay()                      # untimed replay: first-touch costs out of the timed region
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(fns)), t1 - t0


def kernel_profile(fns, repeat=1):
    """Eager run of fns with the library's event profiler (a HIP event pair around each launch on its own stream):
    {kernel: (launches, avg us)}. repeat > 1 re-runs each launch between its events (weights then partly cached)."""
    torch.cuda.synchronize()
    exl3._lib.profile_enable(True, repeat=repeat)
    for f in fns:
        f()
    torch.cuda.synchronize()
    prof = exl3._lib.profile_read()
    exl3._lib.profile_enable(False)
    return prof


# ------------------------------------------------------------------------------------------------ workloads
class MoEWorkload:
    """Routed MoE layer over `copies` layer copies, with `nrout` precomputed routings (fp32 logits on the device)."""

    def __init__(self, name, layers, M, topk, nrout, seed, act, shared=False, bias=None):
        self.name, self.layers, self.M, self.topk = name, layers, M, topk
        t = layers[0]
        self.H, self.I, self.E = t.H, t.I, t.E - (1 if shared else 0)
        self.shared = self.E if shared else -1
        self.act = act
        self.bias = bias
        g = dev_gen(seed)
        self.x = [torch.randn(M, self.H, device="cuda", generator=g).half() for _ in range(nrout)]
        self.logits = [torch.randn(M, self.E, device="cuda", generator=g) for _ in range(nrout)]
        self.i = 0
        # host copy of every routing (for byte / flop accounting)
        self.ids = []
        for lg in self.logits:
            ids, _ = exl3.route_softmax_topk(lg, topk, bias)
            self.ids.append(ids.cpu())
        self.exp_bytes = [proj_bytes(t.projs[0][e]) + proj_bytes(t.projs[1][e]) + proj_bytes(t.projs[2][e])
                          for e in range(t.E)]
        self.gu_bytes = proj_bytes(t.projs[0][0]) + proj_bytes(t.projs[1][0]) + 2 * self.I

    def step_fn(self, j):
        lay = self.layers[j % len(self.layers)]
        r = j % len(self.logits)
        x, lg = self.x[r], self.logits[r]

        def f():
            exl3.moe_forward_logits(x, lg, self.topk, lay, self.act, 0.0, self.shared, bias=self.bias)
        return f

    def experts_used(self, j):
        ids = self.ids[j % len(self.ids)]
        used = [int(e) for e in torch.unique(ids[ids >= 0])]
        return used + ([self.shared] if self.shared >= 0 else [])

    def unique(self, j):
        return len(self.experts_used(j))

    def bytes_per_step(self, j):
        """Algorithmic HBM bytes: the weights of every expert touched once, activations in and out."""
        return sum(self.exp_bytes[e] for e in self.experts_used(j)) + 2 * self.M * self.H + 4 * self.M * self.H

    def flops_per_step(self, j):
        ids = self.ids[j % len(self.ids)]
        pairs = int((ids >= 0).sum()) + (self.M if self.shared >= 0 else 0)
        return 6.0 * pairs * self.H * self.I


def run_moe(wl, steps, label):
    fns = [wl.step_fn(j) for j in range(steps)]
    for f in fns[: min(steps, 4)]:
        f()
    us, _ = graph_time(fns)
    byts = sum(wl.bytes_per_step(j) for j in range(steps)) / steps
    flops = sum(wl.flops_per_step(j) for j in range(steps)) / steps
    gbs = byts / us / 1e3
    r = {"us_per_layer": round(us, 3), "us_per_token": round(us / wl.M, 3), "tokens": wl.M,
         "gbps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
         "tflops": round(flops / us / 1e6, 2), "mfma_frac": round(flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
         "bytes_per_layer": int(byts), "unique_experts": round(sum(wl.unique(j) for j in range(steps)) / steps, 2)}
    log(label, r)
    return r


def run_dense(k, n, K, M, copies, steps, seed, label):
    g = dev_gen(seed)
    lins = [dev_linear(k, n, K, g) for _ in range(copies)]
    x = torch.randn(M, k, device="cuda", generator=g).half()
    y = torch.empty(M, n, dtype=torch.float16, device="cuda")
    fns = [(lambda l=lins[j % copies]: exl3.exl3_gemm(x, l.trellis, y, l.suh, None, l.svh)) for j in range(steps)]
    for f in fns[:4]:
        f()
    us, _ = graph_time(fns)
    byts = k * n * K / 8 + 2 * k + 2 * n + 2 * M * k + 2 * M * n
    gbs = byts / us / 1e3
    r = {"us_per_layer": round(us, 3), "us_per_token": round(us / M, 3), "tokens": M, "gbps": round(gbs, 1),
         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": int(byts), "weight_copies": copies}
    log(label, r)
    return r


def run_mlp(H, I, K, M, copies, steps, seed, label):
    g = dev_gen(seed)
    mlps = []
    for _ in range(copies):
        gt, up, dn = dev_linear(H, I, K, g), dev_linear(H, I, K, g), dev_linear(I, H, K, g)
        mlps.append(exl3.BC_GatedMLP(None, None, None, None, None, None, None, K, False, True, False, True, False,
                                     gt, up, dn, 0.0))
    x = torch.randn(M, H, device="cuda", generator=g).half()
    d = torch.empty(M, H, dtype=torch.float32, device="cuda")
    fns = [(lambda m=mlps[j % copies]: m.run_bszN(x, d)) for j in range(steps)]
    for f in fns[:4]:
        f()
    us, _ = graph_time(fns)
    byts = 3 * (H * I * K / 8) + 2 * (2 * (H + I) + 2 * (I + H)) + 2 * M * H + 4 * M * H
    gbs = byts / us / 1e3
    r = {"us_per_layer": round(us, 3), "us_per_token": round(us / M, 3), "tokens": M, "gbps": round(gbs, 1),
         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": int(byts), "weight_copies": copies}
    log(label, r)
    return r


def zipf_bias(E, s, seed):
    g = torch.Generator().manual_seed(seed)
    rank = torch.randperm(E, generator=g).float()
    return (-s * torch.log(rank + 1)).cuda()


def recorded_traffic(kname):
    """HBM bytes per launch of the headline kernel from its committed rocprofv3 counter summary (FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by what the counter reads for a plain copy of known size); None without
    one. The counters need a profiler run of their own, so the figure is the recorded one, not a live one."""
    path = os.path.join(ROOT, "profiles", f"{kname}_c3_m4_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


# ------------------------------------------------------------------------------------------------ CPU baseline
def cpu_baseline(wl, seconds=12.0):
    """The oracle (NumPy, fp32 accumulation) on a bounded sample of the headline workload: whole layer calls on the
    host cores until ~`seconds` have passed (at least one)."""
    import numpy as np
    O = importlib.import_module("oracle.exl3_oracle")
    lay = wl.layers[0]

    def oproj(p):
        return O.Proj(p.suh.cpu().numpy(), p.svh.cpu().numpy(), trellis=p.trellis.cpu().numpy(), K=p.Ki)

    t_tot, calls = 0.0, 0
    j = 0
    while t_tot < seconds and calls < 64:
        r = j % len(wl.logits)
        ids, w = O.route_softmax_topk(wl.logits[r].cpu().numpy(), wl.topk)
        used = np.unique(ids)
        experts = {int(e): tuple(oproj(lay.projs[q][int(e)]) for q in range(3)) for e in used}
        x = wl.x[r].cpu().numpy()
        t0 = time.perf_counter()
        O.moe_layer(x, experts, ids, w, O.ACT_SILU, 0.0, None, acc=np.float32)
        t_tot += time.perf_counter() - t0
        calls += 1
        j += 1
    us_tok = t_tot * 1e6 / (calls * wl.M)
    return {"value": round(us_tok, 1), "unit": "us/token", "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"{calls} layer calls of the headline workload ({wl.M} tokens each, routing + expert decode + "
                      f"fp32-accumulated matmuls) by the NumPy oracle; BLAS may use every listed core, the trellis "
                      f"decode runs on one"}


# ------------------------------------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="all", help="comma list of c1..c5 to report next to the headline, or none")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 3 plain device copies of MIB MiB each (the HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (every expert resident on one MI355X); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe > 0:
        n = args.copy_probe << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": n, "copy_probe_bytes_written": n, "copies": 3}), flush=True)
        return
    torch.manual_seed(0)
    K, W = args.steps, args.warmup
    log("device", torch.cuda.get_device_name(0))

    # ---- headline: C3 MoE decode layer, 4 tokens per step
    H, I, E, M = 2048, 512, 512, 4
    layers = [dev_experts(E, H, I, 3, 3, 3000 + 97 * c) for c in range(4)]
    wl = MoEWorkload("c3", layers, M, 10, 64, 31, "silu")
    fns = [wl.step_fn(j) for j in range(K)]
    for j in range(W):
        wl.step_fn(j)()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / K
    byts = sum(wl.bytes_per_step(j) for j in range(K)) / K
    us_tok = ms_step * 1e3 / M

    # dominant kernel, timed live with HIP events on the stream it is launched on: the one-launch fused layer kernel
    # (every touched expert's gate, up and down weights, x in, combined rows out) where the layer takes it, else the
    # gate|up GEMV kernel (gate and up weights of every touched expert, x in, activations out)
    nprof = 64
    prof = kernel_profile([wl.step_fn(j) for j in range(nprof)])
    if "moe_fused" in prof:
        kname = "moe_fused"
        k_bytes = sum(wl.bytes_per_step(j) for j in range(nprof)) / nprof
    else:
        kname = "moe_gateup"
        k_bytes = sum(wl.unique(j) * wl.gu_bytes + 2 * M * H + 2 * M * 10 * I for j in range(nprof)) / nprof
    k_n, k_us = prof.get(kname, (0, float("nan")))
    traffic = recorded_traffic(kname)
    achieved = k_bytes / k_us / 1e3
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kname,
                "kernel_us": round(k_us, 3), "launches": k_n, "bytes_per_launch": int(k_bytes),
                "layer_gbps": round(byts / (ms_step * 1e3) / 1e3, 1)}
    log("kernel profile", prof)

    configs = {}
    want = [c.strip() for c in args.configs.split(",")] if args.configs not in ("all", "none") else \
        (["c1", "c2", "c3", "c4", "c5"] if args.configs == "all" else [])
    if "c3" in want:
        for m in (1, 2, 4):
            configs[f"c3_m{m}"] = run_moe(MoEWorkload("c3", layers, m, 10, 64, 40 + m, "silu"), 64, f"c3 M={m}")
    if "c1" in want:
        configs["c1"] = run_dense(4096, 4096, 4, 1, 128, 256, 1000, "c1")
    if "c2" in want:
        for m in (1, 2, 4):
            configs[f"c2_m{m}"] = run_mlp(5376, 21504, 4, m, 6, 48, 2000 + m, f"c2 M={m}")
    if "c4" in want:
        l4 = [dev_experts(160, 5120, 1536, 2, 3, 4000 + c) for c in range(2)]
        wl4 = MoEWorkload("c4", l4, 512, 8, 4, 41, "silu", bias=zipf_bias(160, 1.1, 4100))
        configs["c4"] = run_moe(wl4, 4, "c4")
        del l4, wl4
    if "c5" in want:
        l5 = [dev_experts(257, 7168, 2048, 0, 0, 5000, mixed=True)]
        wl5 = MoEWorkload("c5", l5, 260, 8, 2, 51, "silu", shared=True)
        configs["c5"] = run_moe(wl5, 2, "c5")
        del l5, wl5
    torch.cuda.synchronize()

    cpu = None if args.no_cpu_baseline else cpu_baseline(wl, args.cpu_seconds)
    out = {
        "metric": METRIC, "value": round(us_tok, 3), "unit": "us/token", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "C3 fine-grained MoE decode layer: H=2048, 512 experts (gate/up 2048->512, down "
                               "512->2048), 3.0 bpw EXL3, softmax top-10 routing from fp32 logits, SiLU, 4 tokens "
                               "per step, fresh routing every step, 4 layer copies (2.4 GB) cycled",
                   "hidden": H, "intermediate": I, "experts": E, "topk": 10, "bits": 3, "tokens_per_step": M,
                   "timing": "HIP graph replay of all steps, wall clock", "layer_gbps": roofline["layer_gbps"],
                   "layer_hbm_frac": round(roofline["layer_gbps"] / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
