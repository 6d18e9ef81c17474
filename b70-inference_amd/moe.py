"""Grouped EXL3 MoE on the HIP kernels: expert pointer tables, the routed multi-GEMM, routers, gated MLPs.

Interfaces mirror the reference boundary:
  * moe_forward(x, topk_ids, topk_w, tables, ...) -> out, the exl3xpu_moe::moe_forward op
    (glm/xpu/csrc/exl3_moe.n128.sycl:1380-1439, 1681-1682) over the nine per-projection pointer tables that
    BC_BlockSparseMLP / exl3_moe take (ext-op-inventory.md:1027-1034, 1060-1093)
  * BlockSparseMLP.forward(x, params, out_dtype) -> fp32 routed sum + shared expert, the patched forward of
    glm/xpu/glm_xpu/moe_patch.py:68-94 and dsv41/xpu/dsv_xpu/moe.py:1563-1630
  * BC_GatedMLP(...).run_bszN(x, d) (glm/xpu/glm_xpu/ops.py:157-172), silu_mul / gelu_mul (ext-op-inventory.md:944-956)
  * route_softmax_topk: the fused softmax/top-k router of trellis-serve (trellis-serve.patch:395-441)
  * route_topk / router_logits / routing_ds3_nogroup: scored top-k routing (softmax, sigmoid + bias, sqrt-softplus)
    and the router GEMV from hidden states (glm/xpu/glm_xpu/ops.py:177-193; dsv41/xpu/csrc/dsv_moe_glue.sycl:155-193,
    442-470)
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import (ACT_GELU_TANH, ACT_SILU, EXL3_F16, EXL3_F32, EXL3_WORDS_PLANAR4, EXL3_WORDS_TILE_ORDER, Exl3Error,
                   check, lib, ptr, require_device, stream_of)
from .linear import BC_LinearEXL3

ACTS = {"silu": ACT_SILU, "gelu_tanh": ACT_GELU_TANH, ACT_SILU: ACT_SILU, ACT_GELU_TANH: ACT_GELU_TANH}


class MixedEXL3:
    """An EXL3 projection whose 16x16 tiles carry their own K (1..8): tile i (row-major over [k/16, n/16]) holds
    8 * kmap[i] uint32 words at words[woff[i]:]. A per-projection K is the special case of a constant map."""

    def __init__(self, words: torch.Tensor, kmap: torch.Tensor, woff: torch.Tensor, suh: torch.Tensor,
                 svh: torch.Tensor):
        if kmap.dtype != torch.uint8 or woff.dtype != torch.int32 or words.dtype not in (torch.int32, torch.int16):
            raise Exl3Error("MixedEXL3: words int32, kmap uint8, woff int32 expected")
        self.words, self.kmap, self.woff, self.suh, self.svh = words, kmap, woff, suh, svh
        self.in_features, self.out_features = suh.numel(), svh.numel()
        if kmap.numel() != (self.in_features // 16) * (self.out_features // 16) or woff.numel() != kmap.numel() + 1:
            raise Exl3Error("MixedEXL3: kmap / woff sizes do not match the shape")
        # the kernels stage a tile in 8 * kmap words and fetch it with 16-byte loads at words + woff: K in 1..8,
        # woff the running sum of 8 * kmap from 0, words 16-byte aligned and long enough
        km = kmap.to(torch.int64)
        if kmap.numel() and (int(km.min()) < 1 or int(km.max()) > 8):
            raise Exl3Error("MixedEXL3: every kmap entry must be in 1..8")
        wo = woff.to(torch.int64)
        if int(wo[0]) != 0 or not torch.equal(wo[1:] - wo[:-1], 8 * km):
            raise Exl3Error("MixedEXL3: woff must be the running sum of 8 * kmap starting at 0")
        if words.numel() * words.element_size() < 4 * int(wo[-1]) or words.data_ptr() % 16:
            raise Exl3Error("MixedEXL3: words must hold woff[-1] uint32 words and be 16-byte aligned")
        if kmap.data_ptr() % 4 or not kmap.is_contiguous():
            raise Exl3Error("MixedEXL3: kmap must be contiguous and 4-byte aligned (the kernels read it by dwords)")
        self.K = 0
        self.trellis = words

    def to(self, dev):
        return MixedEXL3(*(t.to(dev) for t in (self.words, self.kmap, self.woff, self.suh, self.svh)))


def _proj_K(p) -> int:
    return 0 if isinstance(p, MixedEXL3) else p.Ki


class ExpertTables:
    """Device tables of E experts: int64 [9, E] = (trellis, suh, svh) addresses of gate, up, down, plus int64 [6, E]
    (kmap, woff) addresses for per-tile-K projections. Holds references to every tensor it points at."""

    def __init__(self, gates, ups, downs):
        if not (len(gates) == len(ups) == len(downs)) or not gates:
            raise Exl3Error("ExpertTables: gate/up/down lists must be non-empty and equally long")
        self.E = len(gates)
        self.projs = (list(gates), list(ups), list(downs))
        Ks = []
        for plist in self.projs:
            ks = {_proj_K(p) for p in plist}
            if len(ks) != 1:
                raise NotImplementedError("ExpertTables: every expert of a projection must share K (or all be per-tile)")
            Ks.append(ks.pop())
        self.K_gate, self.K_up, self.K_down = Ks
        g0, d0 = gates[0], downs[0]
        self.H, self.I = g0.in_features, g0.out_features
        for p in gates + ups:
            if (p.in_features, p.out_features) != (self.H, self.I):
                raise Exl3Error("ExpertTables: gate/up shapes differ")
        for p in downs:
            if (p.in_features, p.out_features) != (self.I, self.H):
                raise Exl3Error("ExpertTables: down shapes differ")
        dev = g0.suh.device
        rows = []
        for plist in self.projs:
            rows.append([p.trellis.data_ptr() for p in plist])
            rows.append([p.suh.data_ptr() for p in plist])
            rows.append([p.svh.data_ptr() for p in plist])
        self.tables = torch.tensor(rows, dtype=torch.int64).to(dev)
        self.kmaps = None
        if 0 in Ks:
            krows = []
            for plist in self.projs:
                krows.append([p.kmap.data_ptr() if isinstance(p, MixedEXL3) else 0 for p in plist])
                krows.append([p.woff.data_ptr() if isinstance(p, MixedEXL3) else 0 for p in plist])
            self.kmaps = torch.tensor(krows, dtype=torch.int64).to(dev)
        # uniform layout (every table row an arithmetic progression over the experts, no per-tile K): the decode
        # kernels then compute an expert's addresses (base + e * stride) instead of loading them
        self.layout = None
        if self.kmaps is None:
            bases, strides = [], []
            for r in rows:
                st = r[1] - r[0] if self.E > 1 else 0
                if any(r[e] - r[0] != e * st for e in range(self.E)):
                    break
                bases.append(r[0])
                strides.append(st)
            else:
                self.layout = (ctypes.c_int64 * 18)(*bases, *strides)

    @classmethod
    def packed(cls, gates, ups, downs):
        """The same experts copied into one contiguous allocation per projection and tensor kind ([E, ...] trellis, suh,
        svh), so every table row is base + e * stride (the layout the decode kernels address without table loads).
        Projections must share K (BC_LinearEXL3)."""
        out = []
        for plist in (gates, ups, downs):
            if any(isinstance(p, MixedEXL3) for p in plist):
                raise NotImplementedError("ExpertTables.packed: per-tile-K projections are not packed")
            tr = torch.stack([p.trellis for p in plist])
            su = torch.stack([p.suh for p in plist])
            sv = torch.stack([p.svh for p in plist])
            out.append([BC_LinearEXL3(tr[e], su[e], sv[e], plist[e].K, None, False, True, None)
                        for e in range(len(plist))])
        return cls(*out)

    def weight_bytes(self, experts) -> int:
        """Trellis + sign-vector bytes of the given expert indices (the algorithmic HBM bytes of reading them)."""
        tot = 0
        for e in experts:
            for p in (self.projs[0][e], self.projs[1][e], self.projs[2][e]):
                tot += p.trellis.numel() * p.trellis.element_size() + 2 * (p.in_features + p.out_features)
                if isinstance(p, MixedEXL3):
                    tot += p.kmap.numel() + 4 * p.woff.numel()
        return tot


def moe_forward(x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, tables: ExpertTables, act=ACT_SILU,
                act_limit: float = 0.0, shared: int = -1, out: torch.Tensor | None = None,
                out_dtype=torch.float32) -> torch.Tensor:
    """out[t] = sum_j topk_w[t, j] * expert_{topk_ids[t, j]}(x[t]) (+ expert `shared` with weight 1), fp32 sums.
    x fp16 [M, H]; topk_ids int32 [M, k] (negative = inactive); topk_w fp32 [M, k]."""
    require_device(x, topk_ids, topk_w)
    if x.dim() != 2 or x.dtype != torch.float16 or x.stride(1) != 1 or x.shape[1] != tables.H:
        raise Exl3Error(f"moe_forward: x must be fp16 [M, {tables.H}] with contiguous rows")
    M = x.shape[0]
    if topk_ids.dtype != torch.int32 or topk_w.dtype != torch.float32:
        raise Exl3Error("moe_forward: topk_ids int32 and topk_w fp32 expected")
    if topk_ids.shape != topk_w.shape or topk_ids.dim() != 2 or topk_ids.shape[0] != M:
        raise Exl3Error("moe_forward: topk_ids / topk_w must be [M, k]")
    topk_ids, topk_w = topk_ids.contiguous(), topk_w.contiguous()
    if out is None:
        out = torch.empty(M, tables.H, dtype=out_dtype, device=x.device)
    if out.dtype not in (torch.float16, torch.float32) or out.stride(1) != 1 or tuple(out.shape) != (M, tables.H):
        raise Exl3Error("moe_forward: out must be fp16/fp32 [M, H] with contiguous rows")
    a = ACTS.get(act)
    if a is None:
        raise NotImplementedError(f"moe_forward: activation {act!r}")
    check(lib().exl3_moe_forward(ptr(x), x.stride(0), M, tables.H, tables.I, ptr(topk_ids), ptr(topk_w),
                                 topk_ids.shape[1], tables.E, ptr(tables.tables), ptr(tables.kmaps), tables.K_gate,
                                 tables.K_up, tables.K_down, a, float(act_limit), int(shared), ptr(out),
                                 out.stride(0), EXL3_F32 if out.dtype == torch.float32 else EXL3_F16, stream_of(x)),
          "moe_forward")
    return out


def moe_forward_blobs(x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, ptrs: torch.Tensor, I: int, K: int,
                      n_experts: int, act=ACT_SILU, act_limit: float = 0.0, out: torch.Tensor | None = None,
                      out_dtype=None, tile_order: bool = False) -> torch.Tensor:
    """exl3xpu_moe::moe_forward(x, topk_ids, topk_w, ptrs, I, K, n_experts) -> [M, H] in x's dtype (unless out_dtype)
    (glm/xpu/csrc/exl3_moe.n128.sycl:1380-1439): the routed layer over one expert blob per expert (ptrs: int64 device
    addresses of blobs in the reference's Geom layout, trellis words in its PLANAR4 order as pack_expert writes them;
    tile_order=True for blobs converted once by blob_unplanarize). x fp16 or bf16: bf16 rows are converted to fp16
    first and the fp32 result rounded once to bf16, the reference kernel's own conversion points (its block loads
    convert x to fp16, its combine stores the fp32 sum in x's dtype)."""
    require_device(x, topk_ids, topk_w, ptrs)
    if x.dim() != 2 or x.dtype not in (torch.float16, torch.bfloat16) or x.stride(1) != 1:
        raise Exl3Error("moe_forward_blobs: x must be fp16 or bf16 [M, H] with contiguous rows")
    if topk_ids.dtype != torch.int32 or topk_w.dtype != torch.float32 or topk_ids.shape != topk_w.shape:
        raise Exl3Error("moe_forward_blobs: topk_ids int32 and topk_w fp32 [M, k] expected")
    if ptrs.dtype != torch.int64 or ptrs.numel() < n_experts:
        raise Exl3Error("moe_forward_blobs: ptrs must be int64 [n_experts]")
    if x.dtype == torch.bfloat16:
        if out is not None:
            raise Exl3Error("moe_forward_blobs: out= is for fp16 x")
        y = moe_forward_blobs(x.half(), topk_ids, topk_w, ptrs, I, K, n_experts, act, act_limit,
                              out_dtype=torch.float32, tile_order=tile_order)
        return y if out_dtype == torch.float32 else y.to(out_dtype or torch.bfloat16)
    M, H = x.shape
    topk_ids, topk_w, ptrs = topk_ids.contiguous(), topk_w.contiguous(), ptrs.contiguous()
    if out is None:
        out = torch.empty(M, H, dtype=out_dtype or x.dtype, device=x.device)
    if out.dtype not in (torch.float16, torch.float32) or out.stride(1) != 1 or tuple(out.shape) != (M, H):
        raise Exl3Error("moe_forward_blobs: out must be fp16/fp32 [M, H] with contiguous rows")
    a = ACTS.get(act)
    if a is None:
        raise NotImplementedError(f"moe_forward_blobs: activation {act!r}")
    check(lib().exl3_moe_forward_blobs(ptr(x), x.stride(0), M, H, int(I), ptr(topk_ids), ptr(topk_w),
                                       topk_ids.shape[1] if topk_ids.dim() == 2 else 0, int(n_experts), ptr(ptrs),
                                       int(K), a, float(act_limit), ptr(out), out.stride(0),
                                       EXL3_F32 if out.dtype == torch.float32 else EXL3_F16,
                                       EXL3_WORDS_TILE_ORDER if tile_order else EXL3_WORDS_PLANAR4, stream_of(x)),
          "moe_forward_blobs")
    return out


def blob_unplanarize(ptrs: torch.Tensor, H: int, I: int, K: int) -> None:
    """Optional: put the reference's expert blobs into tile order in place (K = 3, 5, 6, 7; other K need nothing),
    exactly once; afterwards call moe_forward_blobs(..., tile_order=True). The converted blobs no longer serve the
    reference's kernels."""
    require_device(ptrs)
    if ptrs.dtype != torch.int64:
        raise Exl3Error("blob_unplanarize: ptrs must be int64")
    check(lib().exl3_blob_unplanarize(ptr(ptrs.contiguous()), ptrs.numel(), int(H), int(I), int(K), stream_of(ptrs)),
          "blob_unplanarize")


def moe_forward_logits(x: torch.Tensor, logits: torch.Tensor, k: int, tables: ExpertTables, act=ACT_SILU,
                       act_limit: float = 0.0, shared: int = -1, bias: torch.Tensor | None = None,
                       out: torch.Tensor | None = None, out_dtype=torch.float32, return_routing: bool = False):
    """route_softmax_topk(logits, k, bias) then moe_forward, as one library call. logits fp32 [M, n] over the routed
    experts 0 .. n - 1 of `tables`. Returns out, or (out, ids, w) with return_routing."""
    require_device(x, logits, bias)
    if x.dim() != 2 or x.dtype != torch.float16 or x.stride(1) != 1 or x.shape[1] != tables.H:
        raise Exl3Error(f"moe_forward_logits: x must be fp16 [M, {tables.H}] with contiguous rows")
    M = x.shape[0]
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1 or logits.shape[0] != M:
        raise Exl3Error("moe_forward_logits: logits must be fp32 [M, n] with contiguous rows")
    n = logits.shape[1]
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != n or not bias.is_contiguous()):
        raise Exl3Error("moe_forward_logits: bias must be fp32 [n]")
    if out is None:
        out = torch.empty(M, tables.H, dtype=out_dtype, device=x.device)
    if out.dtype not in (torch.float16, torch.float32) or out.stride(1) != 1 or tuple(out.shape) != (M, tables.H):
        raise Exl3Error("moe_forward_logits: out must be fp16/fp32 [M, H] with contiguous rows")
    a = ACTS.get(act)
    if a is None:
        raise NotImplementedError(f"moe_forward_logits: activation {act!r}")
    ids = torch.empty(M, k, dtype=torch.int32, device=x.device)
    w = torch.empty(M, k, dtype=torch.float32, device=x.device)
    layout = ctypes.cast(tables.layout, ctypes.c_void_p) if tables.layout is not None else None
    check(lib().exl3_moe_forward_logits(ptr(x), x.stride(0), M, tables.H, tables.I, ptr(logits), logits.stride(0), n,
                                        ptr(bias), k, tables.E, ptr(tables.tables), ptr(tables.kmaps), tables.K_gate,
                                        tables.K_up, tables.K_down, a, float(act_limit), int(shared), layout, ptr(ids),
                                        ptr(w), ptr(out), out.stride(0),
                                        EXL3_F32 if out.dtype == torch.float32 else EXL3_F16, stream_of(x)),
          "moe_forward_logits")
    return (out, ids, w) if return_routing else out


def moe_align(topk_ids: torch.Tensor, topk_w: torch.Tensor, E: int, shared: int = -1):
    """(counts int32 [E], pair_tok int32 [P], pair_w fp32 [P], pair_of int32 [M*slots]) as the kernels build them."""
    require_device(topk_ids, topk_w)
    M, k = topk_ids.shape
    slots = k + (1 if shared >= 0 else 0)
    dev = topk_ids.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    pair_tok = torch.full((M * slots,), -1, dtype=torch.int32, device=dev)
    pair_w = torch.zeros(M * slots, dtype=torch.float32, device=dev)
    pair_of = torch.empty(M * slots, dtype=torch.int32, device=dev)
    check(lib().exl3_moe_align(ptr(topk_ids.contiguous()), ptr(topk_w.contiguous()), M, k, E, shared, ptr(counts),
                               ptr(pair_tok), ptr(pair_w), ptr(pair_of), stream_of(topk_ids)), "moe_align")
    return counts, pair_tok, pair_w, pair_of


def route_softmax_topk(logits: torch.Tensor, k: int, bias: torch.Tensor | None = None):
    """softmax(logits + bias) -> top-k (descending, ties to the lower index) -> renormalised weights."""
    require_device(logits, bias)
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise Exl3Error("route_softmax_topk: logits must be fp32 [M, E] with contiguous rows")
    M, E = logits.shape
    ids = torch.empty(M, k, dtype=torch.int32, device=logits.device)
    w = torch.empty(M, k, dtype=torch.float32, device=logits.device)
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != E):
        raise Exl3Error("route_softmax_topk: bias must be fp32 [E]")
    check(lib().exl3_route_softmax_topk(ptr(logits), logits.stride(0), M, E, ptr(bias), k, ptr(ids), ptr(w),
                                        stream_of(logits)), "route_softmax_topk")
    return ids, w


SCORES = {"softmax": 0, "sigmoid": 1, "sqrt_softplus": 2}
ROUTE_RENORM, ROUTE_BIAS_SELECT_ONLY = 1, 2
ROUTER_W = {"he": 0, "eh": 1}


def route_topk(logits: torch.Tensor, k: int, bias: torch.Tensor | None = None, score: str = "softmax",
               renorm: bool = True, scaling: float = 1.0, bias_select_only: bool = False):
    """Top-k routing with a scoring function (exl3_route_topk): softmax (bias ranks, and feeds the weights unless
    bias_select_only), sigmoid (rank by sigmoid + bias, or by the logit without a bias) or sqrt_softplus (rank by
    sqrt(softplus) + bias); weights v * scaling / (sum of picked v + 1e-20) with renorm. Returns (ids int32 [M, k],
    w fp32 [M, k]), picks in descending rank, ties to the lower index."""
    require_device(logits, bias)
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise Exl3Error("route_topk: logits must be fp32 [M, E] with contiguous rows")
    if score not in SCORES:
        raise NotImplementedError(f"route_topk: scoring {score!r}")
    M, E = logits.shape
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != E or not bias.is_contiguous()):
        raise Exl3Error("route_topk: bias must be fp32 [E]")
    ids = torch.empty(M, k, dtype=torch.int32, device=logits.device)
    w = torch.empty(M, k, dtype=torch.float32, device=logits.device)
    flags = (ROUTE_RENORM if renorm else 0) | (ROUTE_BIAS_SELECT_ONLY if bias_select_only else 0)
    check(lib().exl3_route_topk(ptr(logits), logits.stride(0), M, E, ptr(bias), k, SCORES[score], flags,
                                float(scaling), ptr(ids), ptr(w), stream_of(logits)), "route_topk")
    return ids, w


def route_adjusted(logits: torch.Tensor, k: int, bias: torch.Tensor | None = None, mul: torch.Tensor | None = None,
                   res: torch.Tensor | None = None, score: str = "sqrt_softplus", renorm: bool = True,
                   scaling: float = 1.0):
    """Top-k with the reference dsv router's residency terms (exl3_route_adjusted): rank by s * mul + bias +
    max(res, -1e30) (mul, res fp32 [E] or None), weights from s (sigmoid or sqrt_softplus of the logit) as route_topk.
    Returns (ids int32 [M, k], w fp32 [M, k])."""
    require_device(logits, bias, mul, res)
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise Exl3Error("route_adjusted: logits must be fp32 [M, E] with contiguous rows")
    if score not in ("sigmoid", "sqrt_softplus"):
        raise NotImplementedError(f"route_adjusted: scoring {score!r} (sigmoid or sqrt_softplus)")
    M, E = logits.shape
    for name, t in (("bias", bias), ("mul", mul), ("res", res)):
        if t is not None and (t.dtype != torch.float32 or t.numel() != E or not t.is_contiguous()):
            raise Exl3Error(f"route_adjusted: {name} must be fp32 [E]")
    ids = torch.empty(M, k, dtype=torch.int32, device=logits.device)
    w = torch.empty(M, k, dtype=torch.float32, device=logits.device)
    check(lib().exl3_route_adjusted(ptr(logits), logits.stride(0), M, E, ptr(bias), ptr(mul), ptr(res), k,
                                    SCORES[score], ROUTE_RENORM if renorm else 0, float(scaling), ptr(ids), ptr(w),
                                    stream_of(logits)), "route_adjusted")
    return ids, w


def moe_route(logits: torch.Tensor, bias: torch.Tensor, res, ids: torch.Tensor, w: torch.Tensor, want,
              scaling: float) -> None:
    """dsv_moe::moe_route(logits, bias, res, ids, w, want, scaling) (dsv41/xpu/csrc/dsv_moe_glue.sycl:426-439, bound at
    :621-622): s = sqrt(softplus(logit)); ids (in place, int64 or int32) = top-k of s + bias + res; w = s of the picks
    renormalised (+1e-20) * scaling; want (optional, in place) = the plain top-k of s + bias."""
    k = ids.shape[-1]
    pi, pw = route_adjusted(logits, k, bias, None, res, "sqrt_softplus", True, scaling)
    ids.copy_(pi)
    w.copy_(pw)
    if want is not None:
        wi, _ = route_topk(logits, k, bias, "sqrt_softplus", True, scaling)
        want.copy_(wi)


def route_block(logits: torch.Tensor, k: int, bias: torch.Tensor | None = None, mul: torch.Tensor | None = None,
                rows_per_block: int = 1, block_boost: float = 0.0, scaling: float = 1.0):
    """Verify-block routing (exl3_route_block, sqrt_softplus): rows in blocks of rows_per_block, in order; an expert an
    earlier row of the block picked ranks by s * mul * (1 + block_boost) + bias, the others by s * mul + bias; weights
    from s, renormalised and scaled. Returns (ids int32 [M, k], w fp32 [M, k])."""
    require_device(logits, bias, mul)
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise Exl3Error("route_block: logits must be fp32 [M, E] with contiguous rows")
    M, E = logits.shape
    for name, t in (("bias", bias), ("mul", mul)):
        if t is not None and (t.dtype != torch.float32 or t.numel() != E or not t.is_contiguous()):
            raise Exl3Error(f"route_block: {name} must be fp32 [E]")
    ids = torch.empty(M, k, dtype=torch.int32, device=logits.device)
    w = torch.empty(M, k, dtype=torch.float32, device=logits.device)
    check(lib().exl3_route_block(ptr(logits), logits.stride(0), M, E, ptr(bias), ptr(mul), k, int(rows_per_block),
                                 float(block_boost), float(scaling), ptr(ids), ptr(w), stream_of(logits)),
          "route_block")
    return ids, w


def route_fused(x, w0, w1, bias0, bias1, res0, ids0, w0o, want0, ids1, w1o, logits, scaling0, scaling1, mul0=None,
                mul1=None, rows_per_block: int = 1, block_boost: float = 0.0) -> None:
    """dsv_moe::route_fused (dsv41/xpu/csrc/dsv_moe_glue.sycl:476-520, bound at :622-624): the router logits of this
    layer's gate w0 fp16 [E0, H] and optionally the next layer's w1 [E1, H] into logits (fp32, R rows of E0 + E1, in
    place), then sqrt-softplus picks written in place: ids0 / w0o ranked by s * mul0 + bias0 + res0 (the verify-block
    boost instead when rows_per_block > 1, block_boost > 0 and no res0), want0 (optional) the plain top-k of
    s + bias0, and ids1 / w1o the next layer's picks by s * mul1 + bias1."""
    R = x.shape[0]
    E0 = w0.shape[0]
    E1 = 0 if w1 is None else w1.shape[0]
    k = ids0.shape[-1]
    if logits.numel() < R * (E0 + E1) or not logits.is_contiguous():
        raise Exl3Error("route_fused: logits must hold R * (E0 + E1) contiguous fp32 values")
    lv = logits.reshape(-1)[: R * (E0 + E1)].view(R, E0 + E1)
    router_logits(x, w0, E0, "eh", False, out=lv[:, :E0])
    if E1:
        router_logits(x, w1, E1, "eh", False, out=lv[:, E0:])
    S = int(rows_per_block)
    blk = S > 1 and block_boost > 0.0 and R % S == 0

    def rt(lg, bias, res, mul, sc, ids_out, w_out, want_out):
        if blk and res is None:
            pi, pw = route_block(lg, k, bias, mul, S, block_boost, sc)
        else:
            pi, pw = route_adjusted(lg, k, bias, mul, res, "sqrt_softplus", True, sc)
        ids_out.copy_(pi)
        w_out.copy_(pw)
        if want_out is not None:
            wi, _ = route_topk(lg, k, bias, "sqrt_softplus", True, sc)
            want_out.copy_(wi)

    rt(lv[:, :E0], bias0, res0, mul0, scaling0, ids0, w0o, want0)
    if E1:
        rt(lv[:, E0:], bias1, None, mul1, scaling1, ids1, w1o, None)


def router_logits(x: torch.Tensor, weight: torch.Tensor, E: int | None = None, layout: str = "he",
                  round_fp16: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """Router logits fp32 [M, E] = x @ W on the router GEMV (exl3_router_logits). layout "he": weight fp16 [H, >= E]
    (the reference's gate_tensor, columns :E used); "eh": weight fp16 [>= E, H] (a linear layer's weight, rows :E).
    round_fp16 rounds each logit to fp16 precision, as a matmul of two fp16 tensors returns it."""
    require_device(x, weight, out)
    if layout not in ROUTER_W:
        raise Exl3Error(f"router_logits: layout {layout!r}")
    if x.dim() != 2 or x.dtype != torch.float16 or x.stride(1) != 1:
        raise Exl3Error("router_logits: x must be fp16 [M, H] with contiguous rows")
    if weight.dim() != 2 or weight.dtype != torch.float16 or weight.stride(1) != 1:
        raise Exl3Error("router_logits: weight must be fp16 2-D with contiguous rows")
    M, H = x.shape
    if layout == "he":
        if weight.shape[0] != H:
            raise Exl3Error(f"router_logits: weight must be [{H}, E]")
        E = weight.shape[1] if E is None else E
    else:
        if weight.shape[1] != H:
            raise Exl3Error(f"router_logits: weight must be [E, {H}]")
        E = weight.shape[0] if E is None else E
    if out is None:
        out = torch.empty(M, E, dtype=torch.float32, device=x.device)
    if out.dtype != torch.float32 or out.stride(1) != 1 or tuple(out.shape) != (M, E):
        raise Exl3Error("router_logits: out must be fp32 [M, E] with contiguous rows")
    check(lib().exl3_router_logits(ptr(x), x.stride(0), M, H, ptr(weight), weight.stride(0), E, ROUTER_W[layout],
                                   1 if round_fp16 else 0, ptr(out), out.stride(0), stream_of(x)), "router_logits")
    return out


def routing_ds3_nogroup(hidden, gate, scores, bias, topk_indices, topk_weights, scaling_factor, gate_t, act_fn,
                        gate_i8, gate_sb):
    """Sigmoid / noaux_tc top-k routing without groups, in place, as glm/xpu/glm_xpu/ops.py:177-193: logits =
    hidden @ gate[:, :E] rounded to fp16 -> scores; selection by sigmoid + bias (by the logits without a bias); weights
    from the unbiased sigmoid, normalised over the picks (+1e-20) and scaled. gate_t, gate_i8 and gate_sb feed only the
    reference's CUDA deterministic GEMM and are ignored. Inputs other than fp16 are converted to fp16 (the reference
    multiplies them in fp32, then rounds the logits to fp16)."""
    if act_fn != 0:
        raise NotImplementedError("routing_ds3_nogroup: sigmoid routing only (act_fn 0)")
    E = scores.shape[-1]
    k = topk_indices.shape[-1]
    h = hidden.reshape(-1, hidden.shape[-1])
    h = (h if h.dtype == torch.float16 else h.half()).contiguous()
    g = gate if gate.dtype == torch.float16 and gate.stride(-1) == 1 else gate.half().contiguous()
    logits = router_logits(h, g, E=E, layout="he", round_fp16=True)
    scores.copy_(logits.view(scores.shape))
    b = None if bias is None else bias.float().contiguous()
    ids, w = route_topk(logits, k, b, "sigmoid", renorm=True, scaling=float(scaling_factor))
    topk_indices.copy_(ids.view(topk_indices.shape))
    topk_weights.copy_(w.view(topk_weights.shape))


def _act_mul(x, y, z, act, act_limit):
    require_device(x, y, z)
    if x.shape != y.shape or x.numel() != z.numel() or x.dtype != y.dtype or z.dtype != torch.float16:
        raise Exl3Error("act_mul: x, y same shape and dtype, z fp16 with as many elements")
    if not (x.is_contiguous() and y.is_contiguous() and z.is_contiguous()):
        raise Exl3Error("act_mul: tensors must be contiguous")
    dt = EXL3_F16 if x.dtype == torch.float16 else EXL3_F32
    check(lib().exl3_act_mul(ptr(x), ptr(y), ptr(z), x.numel(), dt, act, float(act_limit), stream_of(x)), "act_mul")


def silu_mul(x, y, z, act_limit):
    """z = min(silu(x), L) * clamp(y, -L, L) (L = act_limit, 0 disables), written into z (fp16)."""
    _act_mul(x, y, z, ACT_SILU, act_limit)


def gelu_mul(x, y, z, act_limit=0.0):
    """z = gelu_tanh(x) * y, written into z (fp16)."""
    _act_mul(x, y, z, ACT_GELU_TANH, 0.0)


class BC_GatedMLP:
    """Dense / shared-expert gated MLP: g, u = gate(x), up(x); a = act(g, u); d = down(a). run_bszN(x, d) writes the
    fp32 result into d. Runs as a one-expert table through the grouped kernels (fused activation epilogue).
    Constructor mirrors glm/xpu/glm_xpu/ops.py:157-172 (scratch buffers and fused pointer tables are accepted and
    ignored; gate and up handles are required)."""

    def __init__(self, guh, gu, a, down_xh, gu_ptrs_trellis, gu_ptrs_suh, gu_ptrs_svh, gu_K, gu_mcg, gu_mul1,
                 act_silu, act_gelu, act_relu2, gate, up, down, act_limit):
        if gate is None or up is None:
            raise NotImplementedError("BC_GatedMLP: fused gate/up pointer tables without gate/up handles")
        if act_relu2:
            raise NotImplementedError("BC_GatedMLP: relu2 activation")
        if not (act_silu or act_gelu):
            raise NotImplementedError("BC_GatedMLP: activation must be SiLU or GELU")
        self.gate, self.up, self.down = gate, up, down
        self.act = ACT_SILU if act_silu else ACT_GELU_TANH
        self.act_limit = act_limit
        self.tables = ExpertTables([gate], [up], [down])
        self._ids = {}

    def run_bszN(self, x: torch.Tensor, d: torch.Tensor) -> None:
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype != torch.float16:
            x2 = x2.half()
        x2 = x2.contiguous()
        M = x2.shape[0]
        key = (x2.device, M)
        if key not in self._ids:
            self._ids[key] = (torch.empty(M, 0, dtype=torch.int32, device=x2.device),
                              torch.empty(M, 0, dtype=torch.float32, device=x2.device))
        ids, w = self._ids[key]
        d2 = d.view(-1, d.shape[-1])
        moe_forward(x2, ids, w, self.tables, self.act, self.act_limit, shared=0, out=d2)

    def forward(self, x: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
        d = torch.empty(x.shape[:-1] + (self.down.out_features,), dtype=out_dtype, device=x.device)
        self.run_bszN(x, d)
        return d


class BlockSparseMLP:
    """Routed MoE layer: route (top-k over router logits, optional per-expert bias), grouped routed experts, plus the
    shared expert (weight 1, added after the routed slots). forward returns fp32.

    `experts` holds the routed experts first and, when `has_shared`, the shared expert as the last table entry.
    Router logits come from params["router_logits"] or from `router_weight` on the router GEMV: fp16 [H, E] (layout
    "he", the reference's gate_tensor) or [E, H] ("eh"), optionally rounded to fp16 like a half matmul. Scoring:
    "softmax" (default; the bias ranks and, unless bias_select_only, shifts the softmax), "sigmoid" or
    "sqrt_softplus" (rank by score + bias, weights from the score), renormalised (+1e-20) and scaled by
    routed_scaling."""

    def __init__(self, experts: ExpertTables, num_experts_per_tok: int, has_shared: bool = False, act="silu",
                 act_limit: float = 0.0, router_weight: torch.Tensor | None = None,
                 selection_bias: torch.Tensor | None = None, scoring: str = "softmax", routed_scaling: float = 1.0,
                 renormalize: bool = True, bias_select_only: bool = False, router_layout: str = "he",
                 router_round_fp16: bool = False):
        self.experts = experts
        self.num_experts = experts.E - (1 if has_shared else 0)
        self.num_experts_per_tok = num_experts_per_tok
        self.shared = experts.E - 1 if has_shared else -1
        self.act = ACTS[act]
        self.act_limit = act_limit
        self.router_weight = router_weight
        self.selection_bias = selection_bias
        if scoring not in SCORES:
            raise NotImplementedError(f"BlockSparseMLP: scoring {scoring!r}")
        self.scoring = scoring
        self.routed_scaling = float(routed_scaling)
        self.renormalize = renormalize
        self.bias_select_only = bias_select_only
        self.router_layout = router_layout
        self.router_round_fp16 = router_round_fp16

    def _fused_router(self) -> bool:
        # the one-call path covers softmax ranked and weighted with the bias, renormalised, unscaled
        return (self.scoring == "softmax" and self.renormalize and self.routed_scaling == 1.0 and
                not (self.bias_select_only and self.selection_bias is not None))

    def route(self, x2: torch.Tensor, params=None):
        return route_topk(self.router_logits(x2, params), self.num_experts_per_tok, self.selection_bias, self.scoring,
                          self.renormalize, self.routed_scaling, self.bias_select_only)

    def router_logits(self, x2: torch.Tensor, params=None) -> torch.Tensor:
        logits = None if params is None else params.get("router_logits")
        if logits is None:
            if self.router_weight is None:
                raise Exl3Error("BlockSparseMLP: no router weight and no params['router_logits']")
            return router_logits(x2, self.router_weight, self.num_experts, self.router_layout, self.router_round_fp16)
        return logits.reshape(-1, self.num_experts).float().contiguous()

    def forward(self, x: torch.Tensor, params=None, out_dtype=None) -> torch.Tensor:
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype != torch.float16:
            x2 = x2.half()
        x2 = x2.contiguous()
        if self._fused_router():
            out = moe_forward_logits(x2, self.router_logits(x2, params), self.num_experts_per_tok, self.experts,
                                     self.act, self.act_limit, self.shared, self.selection_bias,
                                     out_dtype=torch.float32)
        else:
            ids, w = self.route(x2, params)
            out = moe_forward(x2, ids, w, self.experts, self.act, self.act_limit, self.shared)
        out = out.view(x.shape[:-1] + (self.experts.H,))
        return out if out_dtype is None else out.to(out_dtype)
