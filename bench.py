#!/usr/bin/env python3
"""Benchmark of the EXL3 quantized-linear + MoE-expert hot path on one MI355X.

Headline: the largest layer, C5 below. One step = one layer call: 4 decode rows and a 256-row prefill chunk routed
top-8 over 256 experts (+ 1 shared expert), per-tile 1/2-bit weights (1.62 bpw), in one library call
(moe_forward). Timed as a HIP graph of exactly --steps steps (--warmup steps run eagerly first): one untimed replay,
then the median of 5 timed replays; steps cycle through fresh routings. value = microseconds per token (lower is
better). Prints one JSON line.

Workloads (seeded synthetic EXL3 tensors generated on the device; parity is tested against the oracle separately):
  C1  dense linear 4096 -> 4096, K=4, 1 token (128 weight copies cycled: beyond the 256 MB Infinity Cache)
  C2  dense MLP 5376 <-> 21504, K=4, GELU-tanh gate, 1 / 2 / 4 tokens
  C3  MoE decode layer H=2048, 512 experts of I=512, K=3, top-10 softmax, SiLU, 1 / 2 / 4 tokens
  C4  MoE prefill layer H=5120, 160 experts of I=1536, gate/up K=2 + down K=3, top-8 softmax over logits + Zipf(1.1)
      expert bias, 512 tokens
  C5  MoE layer H=7168, 256 experts of I=2048 + 1 shared, per-tile K in {1, 2} (38/62), top-8, 4 decode + 256
      prefill rows in one call                                                                       (headline)

Every config reports: time per layer and per token (graph replay) and the eager single-call latency; what the timed
region holds; algorithmic bytes and FLOP per layer and the HBM / fp16-MFMA
fractions they imply; the library's kernels per step with their event-timed durations; a roofline block for its
dominant kernel (the kernel with the most time per step: its algorithmic bytes or FLOP per launch over its average
launch duration, HIP events on the launch stream); and the CPU baseline (the oracle on this host, bounded sample).
"""
from __future__ import annotations

import argparse
import glob
import importlib
import json
import math
import os
import statistics
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "EXL3 MoE layer µs/token + achieved HBM GB/s (% of peak), 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
VALU_PEAK_LANE_OPS = 256 * 64 * 2.4e9           # 256 CUs x 4 SIMDs x 16 lanes per clock x 2.4 GHz
MFMA_ROWS = 64                                  # the library's MFMA row block (kMfmaRows) and its row classes

exl3 = importlib.import_module("b70-inference_amd")


def log(*a):
    print("bench:", *a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------------ weights
def dev_gen(seed):
    return torch.Generator(device="cuda").manual_seed(int(seed))


def _signs(n, g, scale=1.0):
    return ((torch.randint(0, 2, (n,), device="cuda", generator=g).float() * 2 - 1) * scale).half()


def dev_linear(k, n, K, g):
    tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda", generator=g)
    return exl3.BC_LinearEXL3(tr, _signs(k, g), _signs(n, g, float(torch.tensor(1.0 / math.sqrt(k)).half())), K, None,
                              False, True, None)


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
    words = torch.randint(-(2 ** 31), 2 ** 31, (int(woff[-1]),), dtype=torch.int64, device="cuda",
                          generator=g).to(torch.int32)
    return exl3.MixedEXL3(words, kmap, woff.to(torch.int32), _signs(k, g),
                          _signs(n, g, float(torch.tensor(1.0 / math.sqrt(k)).half())))


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


def weight_bytes(p):
    """Algorithmic bytes of one projection: its trellis words (per-tile K: 32 K bytes per tile, no maps) and its two
    fp16 sign vectors."""
    if isinstance(p, exl3.MixedEXL3):
        tw = int(p.woff[-1]) * 4
    else:
        tw = p.trellis.numel() * p.trellis.element_size()
    return tw + 2 * (p.in_features + p.out_features)


# ------------------------------------------------------------------------------------------------ timing
def eager_time(fns):
    """Eager single-call latency: each fn called once between two device synchronisations, host wall clock (launch
    overhead included); microseconds, the median over the calls."""
    ts = []
    for f in fns:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        f()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e6)
    return statistics.median(ts)


def graph_time(fns, reps=1):
    """Capture fns (in order) into one HIP graph and replay it `reps` times (after an untimed replay), each replay timed
    on its own: us per fn call, the median over the replays."""
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / len(fns))
    return sorted(ts)[len(ts) // 2]


def kernel_profile(fns, warm=()):
    """Eager run of fns with the library's event profiler (a HIP event pair recorded with each dispatch on its own
    stream): {kernel: (launches, avg us)}. The `warm` calls run first, unprofiled (eager launches of microsecond
    kernels right after a graph replay otherwise read slow)."""
    for f in warm:
        f()
    torch.cuda.synchronize()
    exl3._lib.profile_enable(True)
    for f in fns:
        f()
    torch.cuda.synchronize()
    prof = exl3._lib.profile_read()
    exl3._lib.profile_enable(False)
    return prof


def cpu_info():
    """(cores this process may run on, the oracle's thread count, a description of the host CPU): lscpu's vendor,
    model name, family / model / stepping, sockets and cores per socket, and /proc/cpuinfo's model name."""
    cores = len(os.sched_getaffinity(0))
    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    proc = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    proc = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    keys = ("Vendor ID", "Model name", "CPU family", "Model", "Stepping", "Socket(s)", "Core(s) per socket",
            "Thread(s) per core", "CPU(s)")
    model = "; ".join(f"{k}: {fields[k]}" for k in keys if k in fields)
    if proc:
        model += f"; /proc/cpuinfo model name: {proc}"
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(cores, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else cores
    return cores, threads, model or None


def cpu_time(fn, runs=3):
    """One warm-up call, then the median of `runs` timed calls (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


# ------------------------------------------------------------------------------------------------ workloads
class Dense:
    """C1: one EXL3 linear k -> n over `copies` weight copies."""
    timed_region = "exl3_gemm (input transform, decode GEMV, output transform)"

    def __init__(self, k, n, K, M, copies, seed):
        g = dev_gen(seed)
        self.k, self.n, self.K, self.M = k, n, K, M
        self.lins = [dev_linear(k, n, K, g) for _ in range(copies)]
        self.x = torch.randn(M, k, device="cuda", generator=g).half()
        self.y = torch.empty(M, n, dtype=torch.float16, device="cuda")

    def step_fn(self, j):
        lin = self.lins[j % len(self.lins)]
        return lambda: exl3.exl3_gemm(self.x, lin.trellis, self.y, lin.suh, None, lin.svh)

    def bytes_per_step(self, j):
        return self.k * self.n * self.K / 8 + 2 * self.k + 2 * self.n + 2 * self.M * self.k + 2 * self.M * self.n

    def flops_per_step(self, j):
        return 2.0 * self.M * self.k * self.n

    def weights_per_step(self, j):
        return self.k * self.n

    def kernel_work(self, name, j):
        return (self.bytes_per_step(j), self.flops_per_step(j)) if name == "gemv" else None

    def kernel_weights(self, name, j):
        return self.k * self.n if name == "gemv" else None

    def cpu(self, O, np):
        lin = self.lins[0]
        tr, su, sv = lin.trellis.cpu().numpy(), lin.suh.cpu().numpy(), lin.svh.cpu().numpy()
        x = self.x.cpu().numpy()
        return cpu_time(lambda: O.Proj(su, sv, trellis=tr, K=self.K)(x, np.float16)), self.M, "one layer call"


class Mlp:
    """C2: dense gated MLP H <-> I (the fused decode layer with one always-on expert)."""
    timed_region = "BC_GatedMLP.run_bszN (gate, up, activation, down in one launch)"

    def __init__(self, H, I, K, M, copies, seed):
        g = dev_gen(seed)
        self.H, self.I, self.K, self.M = H, I, K, M
        self.mlps = []
        for _ in range(copies):
            gt, up, dn = dev_linear(H, I, K, g), dev_linear(H, I, K, g), dev_linear(I, H, K, g)
            self.mlps.append(exl3.BC_GatedMLP(None, None, None, None, None, None, None, K, False, True, False, True,
                                              False, gt, up, dn, 0.0))
        self.x = torch.randn(M, H, device="cuda", generator=g).half()
        self.d = torch.empty(M, H, dtype=torch.float32, device="cuda")

    def step_fn(self, j):
        m = self.mlps[j % len(self.mlps)]
        return lambda: m.run_bszN(self.x, self.d)

    def bytes_per_step(self, j):
        return 3 * self.H * self.I * self.K / 8 + 2 * 3 * (self.H + self.I) + 2 * self.M * self.H + 4 * self.M * self.H

    def flops_per_step(self, j):
        return 6.0 * self.M * self.H * self.I

    def weights_per_step(self, j):
        return 3 * self.H * self.I

    def kernel_work(self, name, j):
        return (self.bytes_per_step(j), self.flops_per_step(j)) if name == "moe_fused" else None

    def kernel_weights(self, name, j):
        return 3 * self.H * self.I if name == "moe_fused" else None

    def cpu(self, O, np):
        m = self.mlps[0]
        ps = [O.Proj(p.suh.cpu().numpy(), p.svh.cpu().numpy(), trellis=p.trellis.cpu().numpy(), K=self.K)
              for p in (m.tables.projs[0][0], m.tables.projs[1][0], m.tables.projs[2][0])]
        x = self.x.cpu().numpy()
        return cpu_time(lambda: O.gated_mlp(x, *ps, O.ACT_GELU_TANH)), self.M, "one layer call"


def mfma_blocks(rows):
    """Row blocks of one expert with `rows` rows in the MFMA path: up to MFMA_ROWS rows each -> class index
    (0: <= 16 rows, 1: <= 32, 2: <= 64) per block."""
    out = []
    for q in range(0, rows, MFMA_ROWS):
        c = min(MFMA_ROWS, rows - q)
        out.append((0 if c <= 16 else 1 if c <= 32 else 2, c))
    return out


class MoE:
    """C3 / C4 / C5: a routed MoE layer over `copies` layer copies and `nrout` precomputed routings."""

    def __init__(self, layers, M, topk, nrout, seed, act, shared=False, bias=None, logits_api=False):
        self.layers, self.M, self.topk = layers, M, topk
        t = layers[0]
        self.H, self.I = t.H, t.I
        self.E = t.E - (1 if shared else 0)
        self.shared = self.E if shared else -1
        self.act, self.bias, self.logits_api = act, bias, logits_api
        self.timed_region = ("moe_forward_logits: routing from the router logits + the layer" if logits_api else
                             "moe_forward on precomputed routing ids and weights (the reference op's boundary, "
                             "moe_forward(x, topk_ids, topk_w, ...)): align, input transform, gate|up, down, combine")
        g = dev_gen(seed)
        self.x = [torch.randn(M, self.H, device="cuda", generator=g).half() for _ in range(nrout)]
        self.logits = [torch.randn(M, self.E, device="cuda", generator=g) for _ in range(nrout)]
        self.routing = [exl3.route_softmax_topk(lg, topk, bias) for lg in self.logits]
        self.ids = [ids.cpu() for ids, _ in self.routing]
        self.exp_bytes = [[weight_bytes(t.projs[q][e]) for q in range(3)] for e in range(t.E)]
        self.out = torch.empty(M, self.H, dtype=torch.float32, device="cuda")

    def step_fn(self, j):
        lay = self.layers[j % len(self.layers)]
        r = j % len(self.logits)
        x, lg = self.x[r], self.logits[r]
        if self.logits_api:
            return lambda: exl3.moe_forward_logits(x, lg, self.topk, lay, self.act, 0.0, self.shared, bias=self.bias,
                                                   out=self.out)
        ids, w = self.routing[r]
        return lambda: exl3.moe_forward(x, ids, w, lay, self.act, 0.0, self.shared, out=self.out)

    def rows_per_expert(self, j):
        ids = self.ids[j % len(self.ids)]
        v = ids[ids >= 0]
        cnt = torch.bincount(v.to(torch.int64), minlength=self.E + (1 if self.shared >= 0 else 0)).tolist()
        if self.shared >= 0:
            cnt[self.shared] = self.M
        return {e: c for e, c in enumerate(cnt) if c > 0}

    def bytes_per_step(self, j):
        """Algorithmic HBM bytes: the weights of every expert touched, once, x in and fp32 rows out."""
        return sum(sum(self.exp_bytes[e]) for e in self.rows_per_expert(j)) + 2 * self.M * self.H + 4 * self.M * self.H

    def flops_per_step(self, j):
        return 6.0 * sum(self.rows_per_expert(j).values()) * self.H * self.I

    def weights_per_step(self, j):
        return 3 * len(self.rows_per_expert(j)) * self.H * self.I

    def unique(self, j):
        return len(self.rows_per_expert(j))

    def kernel_work(self, name, j):
        """(algorithmic bytes, FLOP) of one launch of kernel `name` in step j, or None when not modelled."""
        rpe = self.rows_per_expert(j)
        if name == "moe_fused":
            return self.bytes_per_step(j), self.flops_per_step(j)
        for proj, tag in ((0, "gateup"), (2, "down")):
            if name.startswith(f"moe_{tag}_mfma_r"):
                cl = {"1": 0, "2": 1, "4": 2}[name[-1]]
                experts = {e: sum(c for k, c in mfma_blocks(r) if k == cl) for e, r in rpe.items()}
                experts = {e: r for e, r in experts.items() if r > 0}
                rows = sum(experts.values())
                if proj == 0:      # gate + up weights, xh rows in (two fp16 planes), fp16 down inputs out
                    b = sum(self.exp_bytes[e][0] + self.exp_bytes[e][1] for e in experts) + 4 * rows * self.H + \
                        2 * rows * self.I
                    f = 4.0 * rows * self.H * self.I
                else:              # down weights, fp16 inputs in, fp32 rows out
                    b = sum(self.exp_bytes[e][2] for e in experts) + 2 * rows * self.I + 4 * rows * self.H
                    f = 2.0 * rows * self.H * self.I
                return b, f
        return None

    def kernel_weights(self, name, j):
        """Weights one launch of kernel `name` decodes in step j (a row block decodes its expert's projection once),
        or None when not modelled."""
        rpe = self.rows_per_expert(j)
        if name == "moe_fused":
            return 3 * len(rpe) * self.H * self.I
        for per, tag in ((2, "gateup"), (1, "down")):
            if name.startswith(f"moe_{tag}_mfma_r"):
                cl = {"1": 0, "2": 1, "4": 2}[name[-1]]
                return per * self.H * self.I * sum(1 for r in rpe.values() for k, _ in mfma_blocks(r) if k == cl)
        return None

    def cpu(self, O, np, rows=None):
        """The oracle on rows `rows` of routing 0 (default: all), layer copy 0."""
        import numpy as np_
        lay = self.layers[0]
        x = self.x[0].cpu().numpy()
        ids, w = O.route_softmax_topk(self.logits[0].cpu().numpy(), self.topk,
                                      None if self.bias is None else self.bias.cpu().numpy())
        sel = np_.arange(self.M) if rows is None else np_.asarray(rows)
        used = sorted(set(int(e) for e in np_.unique(ids[sel])) | ({self.shared} if self.shared >= 0 else set()))

        def oproj(p):
            if isinstance(p, exl3.MixedEXL3):
                return O.Proj(p.suh.cpu().numpy(), p.svh.cpu().numpy(), words=p.words.cpu().numpy().view(np_.uint32),
                              kmap=p.kmap.cpu().numpy(), woff=p.woff.cpu().numpy().astype(np_.int64))
            return O.Proj(p.suh.cpu().numpy(), p.svh.cpu().numpy(), trellis=p.trellis.cpu().numpy(), K=p.Ki)

        experts = {e: tuple(oproj(lay.projs[q][e]) for q in range(3)) for e in used}
        ex_list = [experts.get(e) for e in range(self.E)]
        sh = experts.get(self.shared) if self.shared >= 0 else None
        act = O.ACT_SILU

        def run():
            # routing is part of the layer call, as on the GPU
            r_ids, r_w = O.route_softmax_topk(self.logits[0].cpu().numpy()[sel], self.topk,
                                              None if self.bias is None else self.bias.cpu().numpy())
            O.moe_layer(x[sel], ex_list, r_ids, r_w, act, 0.0, sh)
        return cpu_time(run), len(sel), f"{len(sel)} of the {self.M} rows of one layer call"


def measure(name, wl, steps, cpu=True):
    """Graph-replayed time per step over `steps` steps, the kernel breakdown, the dominant kernel's roofline and the
    CPU baseline of one workload."""
    fns = [wl.step_fn(j) for j in range(steps)]
    for f in fns[: min(steps, 4)]:
        f()
    us = graph_time(fns, reps=5)
    eager = eager_time([wl.step_fn(j) for j in range(min(steps, 9))])
    nprof = min(steps, 16)
    prof = kernel_profile([wl.step_fn(j) for j in range(nprof)], [wl.step_fn(nprof + j) for j in range(nprof)])
    byts = sum(wl.bytes_per_step(j) for j in range(steps)) / steps
    flops = sum(wl.flops_per_step(j) for j in range(steps)) / steps
    wts = sum(wl.weights_per_step(j) for j in range(steps)) / steps
    gbs = byts / us / 1e3
    r = {"us_per_layer": round(us, 3), "us_per_token": round(us / wl.M, 3), "tokens": wl.M,
         "timing": "median of 5 timed replays (after an untimed one) of a HIP graph of the steps, per step",
         "timed_region": wl.timed_region, "eager_us_per_call": round(eager, 1),
         "bytes_per_layer": int(byts), "gbps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
         "flop_per_layer": int(flops), "tflops": round(flops / us / 1e6, 2),
         "mfma_frac": round(flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
         "weights_decoded_per_s": float(f"{wts / us * 1e6:.4g}"),
         "kernels": {k: {"launches_per_step": round(n / nprof, 2), "avg_us": round(t, 3)} for k, (n, t) in prof.items()}}
    if isinstance(wl, MoE):
        r["unique_experts"] = round(sum(wl.unique(j) for j in range(steps)) / steps, 2)
    # dominant kernel: the most time per step (for a prefill layer whose row-class kernels run concurrently that is
    # the class of cold experts, with the least matrix work; the layer's own MFMA fraction is reported beside it)
    dom = max(prof.items(), key=lambda kv: kv[1][0] * kv[1][1])[0] if prof else None
    work = [wl.kernel_work(dom, j) for j in range(nprof)] if dom else []
    if work and all(w is not None for w in work):
        k_n, k_us = prof[dom]
        per_launch = k_n / nprof
        kb = sum(w[0] for w in work) / nprof / per_launch
        kf = sum(w[1] for w in work) / nprof / per_launch
        bound = getattr(wl, "bound", "hbm")
        if bound == "mfma":
            ach = kf / k_us / 1e6
            roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4)}
        else:
            ach = kb / k_us / 1e3
            roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(ach / HBM_PEAK_GBS, 4)}
        roof.update({"kernel": dom, "kernel_us": round(k_us, 3), "launches_per_step": round(per_launch, 2),
                     "bytes_per_launch": int(kb), "flop_per_launch": int(kf),
                     "hbm_frac": round(kb / k_us / 1e3 / HBM_PEAK_GBS, 4),
                     "mfma_frac": round(kf / k_us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4)})
        roof["layer_mfma_frac"] = r["mfma_frac"]
        roof["layer_hbm_frac"] = r["hbm_frac"]
        roof["traffic"] = recorded_traffic(dom, name)
        dw = [wl.kernel_weights(dom, j) for j in range(nprof)]
        vpw = recorded_valu(dom, name)
        if vpw is not None and all(w is not None for w in dw):
            wps = sum(dw) / nprof / per_launch / (k_us * 1e-6)
            roof["decode_alu"] = {"valu_lane_ops_per_weight": vpw, "weights_per_s": float(f"{wps:.4g}"),
                                  "achieved": float(f"{wps * vpw:.4g}"), "peak": VALU_PEAK_LANE_OPS,
                                  "unit": "VALU lane-ops/s", "frac": round(wps * vpw / VALU_PEAK_LANE_OPS, 4)}
        r["roofline"] = roof
    log(name, {k: v for k, v in r.items() if k != "kernels"})
    log(name, "kernels", r["kernels"])
    if cpu:
        import numpy as np
        O = importlib.import_module("oracle.exl3_oracle")
        rows = getattr(wl, "cpu_rows", None)
        t, ntok, what = wl.cpu(O, np, rows) if rows is not None else wl.cpu(O, np)
        cores, threads, _ = cpu_info()
        r["cpu_baseline"] = {"value": round(t * 1e6 / ntok, 1), "unit": "us/token", "cores": threads,
                             "affinity_cores": cores, "kind": "port",
                             "sample": f"{what}, oracle (decode + float64 products in C, OpenMP over {threads} "
                                       f"threads), 1 warm-up + median of 3"}
        log(name, "cpu", r["cpu_baseline"])
    return r


def zipf_bias(E, s, seed):
    g = torch.Generator().manual_seed(seed)
    rank = torch.randperm(E, generator=g).float()
    return (-s * torch.log(rank + 1)).cuda()


def recorded_figure(kind, key, kname, workload):
    """A per-kernel figure `key[kname]: value` from the committed rocprofv3 summaries of a workload
    (profiles/*_<workload>_<kind>.md); None without one."""
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", f"*_{workload}_{kind}.md"))):
        with open(path) as f:
            for line in f:
                if line.startswith(f"{key}[{kname}]:"):
                    return float(line.split(":", 1)[1].split()[0])
    return None


def recorded_valu(kname, workload):
    """VALU lane-operations per decoded weight of a kernel (64 x SQ_INSTS_VALU over the weights its launches decode)
    from its committed counter summary; None without one."""
    return recorded_figure("counters", "valu_lane_ops_per_weight", kname, workload)


def recorded_traffic(kname, workload):
    """HBM bytes per launch of a kernel from its committed counter summary (FETCH_SIZE and WRITE_SIZE per dispatch,
    each scaled by what the counter reads for a plain copy of known size); None without one."""
    v = recorded_figure("hbm_traffic", "traffic_bytes_per_launch", kname, workload)
    return None if v is None else int(v)


# ------------------------------------------------------------------------------------------------ configs
def build(name):
    if name == "c1":
        return Dense(4096, 4096, 4, 1, 128, 1000), 256
    if name.startswith("c2_m"):
        m = int(name[4:])
        return Mlp(5376, 21504, 4, m, 6, 2000 + m), 48
    if name.startswith("c3_m"):
        m = int(name[4:])
        layers = [dev_experts(512, 2048, 512, 3, 3, 3000 + 97 * c) for c in range(4)]
        return MoE(layers, m, 10, 64, 40 + m, "silu", logits_api=True), 64
    if name == "c4":
        layers = [dev_experts(160, 5120, 1536, 2, 3, 4000 + c) for c in range(2)]
        wl = MoE(layers, 512, 8, 4, 41, "silu", bias=zipf_bias(160, 1.1, 4100))
        wl.bound, wl.cpu_rows = "mfma", list(range(64))
        # 16 steps per graph, as for C5: per-step time at 4 / 8 / 16 / 32 steps per graph measured 620-676 / 609 / 602
        # / 600 us (the replay's own start-up cost amortised over the steps)
        return wl, 16
    if name == "c5":
        wl = c5_workload()
        return wl, 4
    raise ValueError(name)


def c5_workload(nrout=4):
    wl = MoE([dev_experts(257, 7168, 2048, 0, 0, 5000, mixed=True)], 260, 8, nrout, 51, "silu", shared=True)
    wl.cpu_rows = list(range(4)) + list(range(4, 260, 21))     # the 4 decode rows and 12 prefill rows
    return wl


# ------------------------------------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="all", help="comma list of c1, c2, c3, c4, c5 to report, or none")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 3 plain device copies of MIB MiB each (the HBM counter calibration) and exit")
    ap.add_argument("--only", default=None, help="run just this one workload eagerly (--steps calls; profiling)")
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
    if args.only:
        wl, _ = build(args.only)
        for j in range(args.steps):
            wl.step_fn(j)()
        torch.cuda.synchronize()
        names = ["gemv", "moe_fused"] + [f"moe_{t}_mfma_r{c}" for t in ("gateup", "down") for c in (1, 2, 4)]
        dec, work = {}, {}
        for n in names:
            w = [wl.kernel_weights(n, j) for j in range(args.steps)]
            if all(v is not None for v in w) and sum(w) > 0:
                dec[n] = sum(w) / args.steps
                kw = [wl.kernel_work(n, j) for j in range(args.steps)]
                work[n] = [sum(b for b, _ in kw) / args.steps, sum(f for _, f in kw) / args.steps]
        print(json.dumps({"only": args.only, "calls": args.steps, "decoded_weights_per_call": dec,
                          "algorithmic_bytes_flop_per_call": work}), flush=True)
        return
    torch.manual_seed(0)
    K, W = args.steps, args.warmup
    log("device", torch.cuda.get_device_name(0))

    # ---- headline: C5, 260 rows per step
    wl = c5_workload()
    fns = [wl.step_fn(j) for j in range(K)]
    for j in range(W):
        wl.step_fn(j)()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    g.replay()                       # untimed replay: first-launch costs of the graph stay out of the timing
    torch.cuda.synchronize()
    walls = []
    for _ in range(5):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
    del g
    wall = statistics.median(walls)
    log("headline replays (s)", [round(w, 5) for w in walls])
    ms_step = wall * 1e3 / K
    us_tok = ms_step * 1e3 / wl.M
    byts = sum(wl.bytes_per_step(j) for j in range(K)) / K
    wl_region = wl.timed_region
    c5 = measure("c5", wl, min(K, 16), cpu=not args.no_cpu_baseline)
    roofline = dict(c5.get("roofline", {}))
    if roofline:
        roofline["traffic"] = recorded_traffic(roofline["kernel"], "c5")
    roofline["layer_gbps"] = round(byts / (ms_step * 1e3) / 1e3, 1)
    cpu = c5.pop("cpu_baseline", None)
    _, _, model = cpu_info()
    if cpu:
        cpu["model"] = model
    del wl, fns
    torch.cuda.empty_cache()

    configs = {"c5": c5}
    want = [c.strip() for c in args.configs.split(",")] if args.configs not in ("all", "none") else \
        (["c1", "c2", "c3", "c4"] if args.configs == "all" else [])
    names = [n for c in want for n in ((c,) if c in ("c1", "c4") else (f"{c}_m1", f"{c}_m2", f"{c}_m4"))
             if c != "c5"]
    for n in names:
        w, steps = build(n)
        configs[n] = measure(n, w, steps, cpu=not args.no_cpu_baseline)
        del w
        torch.cuda.empty_cache()
    torch.cuda.synchronize()

    out = {
        "metric": METRIC, "value": round(us_tok, 3), "unit": "us/token", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "MoE layer H=7168, 256 routed experts of I=2048 + 1 shared expert, per-tile 1/2-bit "
                               "EXL3 weights (38/62, 1.62 bpw), softmax top-8, SiLU; 260 rows per step (4 decode + "
                               "256 prefill) in one call, fresh routing every step",
                   "hidden": 7168, "intermediate": 2048, "experts": 256, "shared_experts": 1, "topk": 8,
                   "bits": 1.62, "rows_per_step": 260,
                   "timing": "HIP graph of all steps: one untimed replay, then the median of 5 timed replays "
                             "(each bracketed by device synchronisations, host wall clock)",
                   "timed_region": wl_region, "eager_us_per_call": c5["eager_us_per_call"],
                   "layer_gbps": roofline["layer_gbps"],
                   "layer_hbm_frac": round(roofline["layer_gbps"] / HBM_PEAK_GBS, 4), "host_cpu": model},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
