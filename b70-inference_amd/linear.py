"""EXL3 linear layer on the HIP kernels: the exllamav3 ext ops of the linear path and the BC_LinearEXL3 shim.

Interfaces mirror the reference boundary:
  * BC_LinearEXL3(trellis, suh, svh, K, bias, mcg, mul1, xh) with run(x, y) / run_alloc(x, out_features, output_fp32)
    (glm/xpu/glm_xpu/ops.py:34-88; ext-op-inventory.md:471-496)
  * exl3_gemm(A, B, C, suh, A_had, svh, force_shape_idx, mcg, mul1, force_num_sms) (ext-op-inventory.md:498-557)
  * exl3_mgemm(A, B, C, suh, A_had, svh, indices, weights, K, force_shape_idx, mcg, mul1, min_index, max_index,
    force_num_sms, num_tokens, ...) over int64 tables of device addresses (ext-op-inventory.md:664-685, 1104-1119)
  * reconstruct / reconstruct_slice (ext-op-inventory.md:597-612), exl3_reconstruct (glm/xpu/csrc/exl3_ops.sycl:539-555)
  * had_r_128(input, output, pre_scale, post_scale, scale) (ext-op-inventory.md:576-595)
  * linear(x, trellis, suh[S, k], svh, shard_of_nb, group_bounds, K, cb, small_m_max, slice_n): the fused
    multi-projection linear of the XPU library (glm/xpu/csrc/exl3_ops.sycl:651-757, bound at :789-790); fuse_linears
    builds its operands from several BC_LinearEXL3 that share the input
Tensors live on the GPU; every op is asynchronous on the current stream and writes its output in place.
"""
from __future__ import annotations

import torch

from ._lib import EXL3_F16, EXL3_F32, Exl3Error, check, lib, ptr, require_device, stream_of

CB_MUL1 = 2


def _cb(mcg: bool, mul1: bool) -> int:
    if mcg:
        raise NotImplementedError("exl3mi: only the mul1 codebook is implemented (mcg requested)")
    if not mul1:
        raise NotImplementedError("exl3mi: only the mul1 codebook is implemented (3inst requested)")
    return CB_MUL1


def _K_of(trellis: torch.Tensor, K=None) -> int:
    if trellis.dim() != 3 or trellis.dtype != torch.int16:
        raise Exl3Error(f"trellis must be int16 [k/16, n/16, 16K], got {tuple(trellis.shape)} {trellis.dtype}")
    Kt = trellis.shape[-1] / 16
    if K is not None and float(K) != Kt:
        raise Exl3Error(f"K={K} does not match trellis.shape[-1]={trellis.shape[-1]}")
    if Kt != int(Kt):
        raise NotImplementedError("exl3mi: half-integer bitrates are not supported")
    return int(Kt)


def exl3_reconstruct(trellis: torch.Tensor, w: torch.Tensor, n0: int, K: int, cb: int = CB_MUL1) -> None:
    """w[:, :] = W_hat[:, n0 : n0 + w.shape[1]] (fp16, Hadamard domain); exl3xpu_C::exl3_reconstruct."""
    require_device(trellis, w)
    if w.dtype != torch.float16 or w.dim() != 2 or w.stride(1) != 1:
        raise Exl3Error("reconstruct output must be a 2D fp16 tensor with unit column stride")
    if not trellis.is_contiguous():
        raise Exl3Error("trellis must be contiguous")
    k = trellis.shape[0] * 16
    if w.shape[0] != k:
        raise Exl3Error(f"reconstruct output has {w.shape[0]} rows, trellis has {k}")
    check(lib().exl3_reconstruct(ptr(trellis), k, trellis.shape[1] * 16, int(K), int(cb), int(n0), w.shape[1], ptr(w),
                                 w.stride(0), stream_of(w)), "exl3_reconstruct")


def reconstruct(unpacked: torch.Tensor, packed: torch.Tensor, K, mcg: bool, mul1: bool) -> None:
    """exllamav3 ext reconstruct(unpacked, packed, K, mcg, mul1)."""
    exl3_reconstruct(packed, unpacked, 0, _K_of(packed, K), _cb(mcg, mul1))


def reconstruct_slice(unpacked: torch.Tensor, packed: torch.Tensor, K, mcg: bool, mul1: bool, n_offset: int) -> None:
    """exllamav3 ext reconstruct_slice(unpacked, packed, K, mcg, mul1, n_offset)."""
    exl3_reconstruct(packed, unpacked, n_offset, _K_of(packed, K), _cb(mcg, mul1))


def reconstruct_had_slice(unpacked: torch.Tensor, packed: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K,
                          mcg: bool, mul1: bool, n_offset: int) -> None:
    """exllamav3 ext reconstruct_had_slice(unpacked, packed, suh, svh, K, mcg, mul1, n_offset): unpacked fp16
    [k, n_slice] = the original-basis weight diag(suh) Hblk W_hat Hblk diag(svh) for columns n_offset .. + n_slice,
    with svh the slice's signs (the caller passes svh[n_offset:], as the reference does). x @ unpacked is the
    linear's output for those columns."""
    require_device(unpacked, packed, suh, svh)
    cb = _cb(mcg, mul1)
    K = _K_of(packed, K)
    if unpacked.dtype != torch.float16 or unpacked.dim() != 2 or unpacked.stride(1) != 1:
        raise Exl3Error("reconstruct_had_slice: unpacked must be a 2D fp16 tensor with unit column stride")
    if not packed.is_contiguous():
        raise Exl3Error("reconstruct_had_slice: trellis must be contiguous")
    k, n_slice = packed.shape[0] * 16, unpacked.shape[1]
    if unpacked.shape[0] != k or suh.numel() != k or svh.numel() < n_slice:
        raise Exl3Error("reconstruct_had_slice: unpacked [k, n_slice], suh [k] and svh [>= n_slice] expected")
    if suh.dtype != torch.float16 or svh.dtype != torch.float16:
        raise Exl3Error("reconstruct_had_slice: suh / svh must be fp16")
    check(lib().exl3_reconstruct_had_slice(ptr(packed), k, packed.shape[1] * 16, K, cb, ptr(suh.contiguous()),
                                           ptr(svh.contiguous()), int(n_offset), n_slice, ptr(unpacked),
                                           unpacked.stride(0), stream_of(unpacked)), "reconstruct_had_slice")


def had_r_128(input: torch.Tensor, output: torch.Tensor, pre_scale, post_scale, scale: float) -> None:
    """Blockwise H128 * scale / sqrt(128) with optional fp16 pre/post scales (pre wins), written into output."""
    require_device(input, output, pre_scale, post_scale)
    if input.shape != output.shape or input.dim() != 2:
        raise Exl3Error("had_r_128: input and output must be 2D with equal shapes")
    if input.dtype != output.dtype or input.dtype not in (torch.float16, torch.float32):
        raise Exl3Error("had_r_128: input/output must both be fp16 or both fp32")
    if input.stride(1) != 1 or output.stride(1) != 1:
        raise Exl3Error("had_r_128: rows must be contiguous")
    for v in (pre_scale, post_scale):
        if v is not None and (v.dtype != torch.float16 or v.numel() != input.shape[1] or not v.is_contiguous()):
            raise Exl3Error("had_r_128: scales must be contiguous fp16 [cols]")
    dt = EXL3_F16 if input.dtype == torch.float16 else EXL3_F32
    check(lib().exl3_had_r_128(ptr(input), input.stride(0), ptr(output), output.stride(0), input.shape[0],
                               input.shape[1], dt, ptr(pre_scale), ptr(post_scale), float(scale), stream_of(input)),
          "had_r_128")


def exl3_gemm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, suh: torch.Tensor, A_had, svh: torch.Tensor,
              force_shape_idx: int = -1, mcg: bool = False, mul1: bool = True, force_num_sms: int = 0) -> int:
    """C = Hn(Hk(A * suh) @ W_hat) * svh; A fp16 [..., k] contiguous, C fp16/fp32 [..., n]. Returns 0 (kernel tag)."""
    require_device(A, B, C, suh, svh)
    K = _K_of(B)
    cb = _cb(mcg, mul1)
    k, n = B.shape[0] * 16, B.shape[1] * 16
    if A.dtype != torch.float16 or A.shape[-1] != k:
        raise Exl3Error(f"exl3_gemm: A must be fp16 [..., {k}]")
    if C.shape[-1] != n or C.dtype not in (torch.float16, torch.float32):
        raise Exl3Error(f"exl3_gemm: C must be fp16/fp32 [..., {n}]")
    if not A.is_contiguous() or not B.is_contiguous() or not C.is_contiguous():
        raise Exl3Error("exl3_gemm: A, B and C must be contiguous")
    if suh.dtype != torch.float16 or svh.dtype != torch.float16 or suh.numel() != k or svh.numel() != n:
        raise Exl3Error("exl3_gemm: suh/svh must be fp16 [k] / [n]")
    m = A.numel() // k
    if C.numel() // n != m:
        raise Exl3Error("exl3_gemm: A and C row counts differ")
    dt = EXL3_F32 if C.dtype == torch.float32 else EXL3_F16
    check(lib().exl3_gemm(ptr(A), k, m, k, ptr(B), n, K, ptr(C), n, dt, ptr(suh.contiguous()), ptr(A_had),
                          ptr(svh.contiguous()), cb, stream_of(A)), "exl3_gemm")
    return 0


def exl3_gemm_noalloc(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor) -> None:
    """exl3_gemm for up to 8 rows with no allocation in the library (its scratch is a fixed per-device array); same
    results as exl3_gemm bit for bit. Calls on one device must not overlap in time."""
    require_device(A, B, C, suh, svh)
    K = _K_of(B)
    k, n = B.shape[0] * 16, B.shape[1] * 16
    if A.dtype != torch.float16 or A.shape[-1] != k or not A.is_contiguous():
        raise Exl3Error(f"exl3_gemm_noalloc: A must be contiguous fp16 [..., {k}]")
    if C.shape[-1] != n or C.dtype not in (torch.float16, torch.float32) or not C.is_contiguous():
        raise Exl3Error(f"exl3_gemm_noalloc: C must be contiguous fp16/fp32 [..., {n}]")
    m = A.numel() // k
    if C.numel() // n != m:
        raise Exl3Error("exl3_gemm_noalloc: A and C row counts differ")
    dt = EXL3_F32 if C.dtype == torch.float32 else EXL3_F16
    check(lib().exl3_gemm_noalloc(ptr(A), k, m, k, ptr(B.contiguous()), n, K, ptr(C), n, dt, ptr(suh.contiguous()),
                                  ptr(svh.contiguous()), CB_MUL1, stream_of(A)), "exl3_gemm_noalloc")


def exl3_mgemm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, suh: torch.Tensor, A_had, svh: torch.Tensor,
               indices, weights, K, force_shape_idx: int = -1, mcg: bool = False, mul1: bool = True,
               min_index: int = -1, max_index: int = -1, force_num_sms: int = 0, num_tokens: int = 1,
               size_n_list=None, c_ptrs=None, n_stride_list=None, had_src_list=None, num_had_src: int = 0) -> int:
    """Multi-matrix EXL3 linear (exllamav3 ext exl3_mgemm). B, suh, svh: int64 device tensors holding one trellis /
    suh / svh address per matrix (e.g. from `mgemm_tables`). A fp16 [a_batches, m, k] with a_batches 1 (broadcast),
    the slot count or num_tokens. Slot j runs matrix indices[j] (indices int64, any shape, flattened; without indices
    slot j runs matrix j); min_index >= 0 keeps only indices in [min_index, max_index), rebased. Negative (or out of
    range) indices skip the slot. Without weights C [slots, m, n] receives each slot's result (skipped slots keep
    their C); with weights ([slots], converted to fp16 as the reference stores them) C [num_tokens, m, n] receives each
    token's weighted sum over its slots in slot order (fp32). A_had is accepted and not used (the input transform is
    fused). The sliced mode (size_n_list, c_ptrs, n_stride_list, had_src_list) is not provided. Returns 0."""
    if size_n_list is not None or c_ptrs is not None or n_stride_list is not None or had_src_list is not None \
            or num_had_src:
        raise NotImplementedError("exl3_mgemm: the sliced mode (size_n_list / c_ptrs / had_src_list) is not provided")
    require_device(A, B, C, suh, svh, indices, weights)
    cb = _cb(mcg, mul1)
    Ki = int(K)
    if float(K) != Ki:
        raise Exl3Error(f"exl3_mgemm: K={K} must be a whole number of bits")
    for name, t in (("B", B), ("suh", suh), ("svh", svh)):
        if t.dtype != torch.int64 or t.numel() != B.numel():
            raise Exl3Error(f"exl3_mgemm: {name} must be an int64 address table of {B.numel()} entries")
    if A.dtype != torch.float16 or not A.is_contiguous() or A.dim() not in (2, 3):
        raise Exl3Error("exl3_mgemm: A must be contiguous fp16 [a_batches, m, k] or [m, k]")
    A3 = A if A.dim() == 3 else A.unsqueeze(0)
    a_batches, m, k = A3.shape
    if C.dtype not in (torch.float16, torch.float32) or not C.is_contiguous() or C.dim() != 3 or C.shape[1] != m:
        raise Exl3Error(f"exl3_mgemm: C must be contiguous fp16/fp32 [batches, {m}, n]")
    n = C.shape[2]
    idx = None
    if indices is not None:
        idx = indices.reshape(-1).to(torch.int64).contiguous()
        slots = idx.numel()
    else:
        slots = B.numel() if weights is not None else C.shape[0]
    w = None
    if weights is not None:
        w = weights.reshape(-1).to(torch.float16).contiguous()
        if w.numel() != slots:
            raise Exl3Error(f"exl3_mgemm: weights must have one entry per slot ({slots})")
        if C.shape[0] != num_tokens:
            raise Exl3Error(f"exl3_mgemm: weighted C must be [num_tokens={num_tokens}, m, n]")
    elif C.shape[0] != slots:
        raise Exl3Error(f"exl3_mgemm: C must be [slots={slots}, m, n]")
    dt = EXL3_F32 if C.dtype == torch.float32 else EXL3_F16
    check(lib().exl3_mgemm(ptr(A3), a_batches, m, k, ptr(B.contiguous()), ptr(suh.contiguous()),
                           ptr(svh.contiguous()), B.numel(), n, Ki, cb, ptr(idx), slots, ptr(w), num_tokens,
                           min_index, max_index, ptr(C), dt, stream_of(A)), "exl3_mgemm")
    return 0


def mgemm_tables(linears, device=None):
    """int64 address tables (trellis, suh, svh) of BC_LinearEXL3 objects of one shape and bitrate, for exl3_mgemm.
    The tables hold raw addresses: the linears' tensors must outlive every call that uses them."""
    if not linears:
        raise Exl3Error("mgemm_tables: no linears")
    shape, K = tuple(linears[0].trellis.shape), linears[0].Ki
    for L in linears:
        if tuple(L.trellis.shape) != shape or L.Ki != K:
            raise Exl3Error("mgemm_tables: every matrix must have the same shape and K")
        for t in (L.trellis, L.suh, L.svh):
            if not t.is_contiguous():
                raise Exl3Error("mgemm_tables: trellis, suh and svh must be contiguous")
    dev = device if device is not None else linears[0].trellis.device
    mk = lambda f: torch.tensor([f(L).data_ptr() for L in linears], dtype=torch.int64).to(dev)  # noqa: E731
    return mk(lambda L: L.trellis), mk(lambda L: L.suh), mk(lambda L: L.svh)


class BC_LinearEXL3:
    """EXL3 linear: y = Had(Had(x * suh) @ W_hat) * svh (+ bias), on the HIP kernels (mul1 codebook).

    Holds the fields other modules read to build pointer tables (trellis, suh, svh, K, bias, mcg, mul1, xh), exactly
    as the reference shim does (glm/xpu/glm_xpu/ops.py:34-88)."""

    def __init__(self, trellis, suh, svh, K, bias, mcg, mul1, xh):
        self.trellis = trellis
        self.suh = suh
        self.svh = svh
        self.K = K
        self.bias = bias
        self.mcg = mcg
        self.mul1 = mul1
        self.xh = xh
        self.cb = _cb(mcg, mul1)
        self.Ki = _K_of(trellis, K)
        self.in_features = trellis.shape[0] * 16
        self.out_features = trellis.shape[1] * 16

    def run(self, x: torch.Tensor, y: torch.Tensor) -> None:
        """x fp16 [..., k] -> y (fp16 or fp32, preallocated) [..., n]."""
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.float16:
            x2 = x2.half()
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        y2 = y.view(-1, self.out_features)
        if x2.shape[0] == 0:
            return
        exl3_gemm(x2, self.trellis, y2, self.suh, self.xh, self.svh, -1, self.mcg, self.mul1, 0)
        if self.bias is not None:
            y2.add_(self.bias)

    def run_alloc(self, x: torch.Tensor, out_features: int, output_fp32: bool) -> torch.Tensor:
        y = torch.empty(x.shape[:-1] + (out_features,), dtype=torch.float if output_fp32 else torch.half,
                        device=x.device)
        if out_features == 0:
            return y
        self.run(x.reshape(-1, x.shape[-1]), y.view(-1, out_features))
        return y


def linear(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, shard_of_nb: torch.Tensor,
           group_bounds, K: int, cb: int = CB_MUL1, small_m_max: int = 8, slice_n: int = 16384,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """exl3xpu_C::linear: y[..., g0:g1] = x @ W_s for the S projections (shards) whose trellises are concatenated
    along the columns; suh fp16 [S, k] (one input sign vector per shard), svh fp16 [n], shard_of_nb int32 [n / 128]
    (device), group_bounds the S + 1 column boundaries. Returns fp16 [..., n] (or writes `out`, fp16 / fp32).
    small_m_max and slice_n tune the reference's own path choice and slicing; the library picks its paths itself."""
    require_device(x, trellis, suh, svh, shard_of_nb, out)
    Ki = _K_of(trellis, K)
    if cb != CB_MUL1:
        raise NotImplementedError(f"exl3mi: codebook {cb} not supported (mul1 = 2 only)")
    k, n = trellis.shape[0] * 16, trellis.shape[1] * 16
    if suh.dim() == 1:
        suh = suh.view(1, -1)
    S = suh.shape[0]
    if suh.dtype != torch.float16 or suh.shape[1] != k or not suh.is_contiguous():
        raise Exl3Error(f"linear: suh must be contiguous fp16 [S, {k}]")
    if svh.dtype != torch.float16 or svh.numel() != n or not svh.is_contiguous():
        raise Exl3Error(f"linear: svh must be contiguous fp16 [{n}]")
    gb = [int(v) for v in group_bounds]
    if len(gb) != S + 1 or gb[0] != 0 or gb[-1] != n or any(b % 128 for b in gb) or gb != sorted(gb):
        raise Exl3Error(f"linear: group_bounds {gb} must be S + 1 = {S + 1} ascending multiples of 128 from 0 to {n}")
    if S > 1 and (shard_of_nb is None or shard_of_nb.dtype != torch.int32 or shard_of_nb.numel() != n // 128 or
                  not shard_of_nb.is_contiguous()):
        raise Exl3Error(f"linear: shard_of_nb must be contiguous int32 [{n // 128}]")
    if x.shape[-1] != k:
        raise Exl3Error(f"linear: x must be [..., {k}]")
    x2 = x.reshape(-1, k)
    x2 = (x2 if x2.dtype == torch.float16 else x2.half()).contiguous()
    M = x2.shape[0]
    if out is None:
        out = torch.empty(x.shape[:-1] + (n,), dtype=torch.float16, device=x.device)
    if out.dtype not in (torch.float16, torch.float32) or not out.is_contiguous() or out.numel() != M * n:
        raise Exl3Error("linear: out must be contiguous fp16/fp32 [..., n]")
    if M == 0:
        return out
    if not trellis.is_contiguous():
        raise Exl3Error("linear: trellis must be contiguous")
    check(lib().exl3_linear_sharded(ptr(x2), k, M, k, ptr(trellis), n, Ki, ptr(out), n,
                                    EXL3_F32 if out.dtype == torch.float32 else EXL3_F16, ptr(suh), S,
                                    ptr(shard_of_nb) if S > 1 else None, ptr(svh), cb, stream_of(x2)), "linear")
    return out


def fuse_linears(linears):
    """Operands of `linear` for BC_LinearEXL3 projections that share the input (same in_features and K): trellis
    concatenated along the columns, suh stacked [S, k], svh concatenated, shard_of_nb and group_bounds (as the
    reference's fused q|k|v and gate|up setup does, trellis-serve.patch:3705-3716). Returns
    (trellis, suh, svh, shard_of_nb, group_bounds, K)."""
    if not linears:
        raise Exl3Error("fuse_linears: no projections")
    k, K = linears[0].in_features, linears[0].Ki
    for lin in linears:
        if lin.in_features != k or lin.Ki != K:
            raise Exl3Error("fuse_linears: projections must share in_features and K")
        if lin.out_features % 128:
            raise Exl3Error("fuse_linears: every projection's out_features must be a multiple of 128")
    tr = torch.cat([lin.trellis for lin in linears], 1).contiguous()
    suh = torch.stack([lin.suh.half() for lin in linears]).contiguous()
    svh = torch.cat([lin.svh.half() for lin in linears]).contiguous()
    bounds = [0]
    for lin in linears:
        bounds.append(bounds[-1] + lin.out_features)
    sonb = torch.empty(bounds[-1] // 128, dtype=torch.int32)
    for g in range(len(linears)):
        sonb[bounds[g] // 128: bounds[g + 1] // 128] = g
    return tr, suh, svh, sonb.to(tr.device), bounds, K
