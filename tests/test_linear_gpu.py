"""GPU parity of the dense EXL3 linear path against the CPU oracle (same seeded bytes on both sides).

Bars: decoded weights bit-exact (fp16 bit patterns); had_r_128 within one fp16 ulp (the kernel's fp32 butterfly vs the
oracle's exact sum) and 1e-6 relative in fp32; linear outputs within max|y - r| / max|r| <= 2e-3 of the oracle's
float64-accumulated result (the reference's max_rel convention, trellis-serve.patch:3889).
"""
import math

import numpy as np
import pytest
import torch

MAX_REL = 2e-3
pytestmark = pytest.mark.gpu


def max_rel(y, r):
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    return float(np.abs(y - r).max() / np.abs(r).max())


def synth():
    import importlib
    return importlib.import_module("b70-inference_amd.synth")


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("k,n", [(128, 128), (256, 384), (512, 1024)])
def test_reconstruct_bit_exact(exl3, oracle, K, k, n):
    tr, _, _ = synth().linear(k, n, K, 1000 + K)
    w = torch.empty(k, n, dtype=torch.float16, device="cuda")
    exl3.exl3_reconstruct(tr.cuda(), w, 0, K)
    ref = oracle.reconstruct(tr.numpy(), K)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_reconstruct_slice_and_stride(exl3, oracle):
    tr, _, _ = synth().linear(256, 1024, 3, 5)
    buf = torch.zeros(256, 512, dtype=torch.float16, device="cuda")
    exl3.reconstruct_slice(buf[:, 128:384], tr.cuda(), 3, False, True, 256)
    ref = oracle.reconstruct(tr.numpy(), 3, 256, 256)
    got = buf.cpu().numpy()
    assert np.array_equal(got[:, 128:384].view(np.uint16), ref.view(np.uint16))
    assert (got[:, :128] == 0).all() and (got[:, 384:] == 0).all()


def test_reconstruct_full_c1(exl3, oracle):
    """4096 x 4096, K=4 (the single-linear workload): every weight bit-exact."""
    tr, _, _ = synth().linear(4096, 4096, 4, 1001)
    w = torch.empty(4096, 4096, dtype=torch.float16, device="cuda")
    exl3.exl3_reconstruct(tr.cuda(), w, 0, 4)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), oracle.reconstruct(tr.numpy(), 4).view(np.uint16))


@pytest.mark.parametrize("K", [1, 2, 3, 4, 8])
def test_reconstruct_had_slice_matches_dense_weight(exl3, oracle, K):
    """Original-basis weight slices (reconstruct_had_slice, the reference's svh[n_offset:] convention) within one fp16
    ulp of the oracle's float64 diag(suh) Hblk W_hat Hblk diag(svh); columns past the slice untouched; x @ W equals
    the linear's output within the tolerance."""
    k, n = 384, 640
    tr, suh, svh = synth().linear(k, n, K, 1100 + K)
    ref = oracle.dense_weight(tr.numpy(), suh.numpy(), svh.numpy(), K)
    full = None
    for n_off, n_sl in ((0, n), (256, 256), (512, 128)):
        buf = torch.full((k, n_sl + 64), float("nan"), dtype=torch.float16, device="cuda")
        exl3.reconstruct_had_slice(buf[:, :n_sl], tr.cuda(), suh.cuda(), svh[n_off:].cuda(), K, False, True, n_off)
        got = buf.cpu().numpy()
        r = ref[:, n_off:n_off + n_sl]
        ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float64)
        assert (np.abs(got[:, :n_sl].astype(np.float64) - r) <= ulp).all()
        assert np.isnan(got[:, n_sl:]).all()
        if n_off == 0:
            full = got[:, :n_sl].astype(np.float64)
    x = synth().activations(3, k, 1200 + K)
    y = oracle.exl3_linear(x.numpy(), tr.numpy(), suh.numpy(), svh.numpy(), K, np.float32)
    assert max_rel(x.numpy().astype(np.float64) @ full, y) <= MAX_REL


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_had_r_128(exl3, oracle, dtype):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 384, generator=g).to(dtype)
    pre = (torch.randint(0, 2, (384,), generator=g) * 2 - 1).half() * 0.75
    for p, q in ((None, None), (pre, None), (None, pre), (pre, pre)):
        out = torch.empty_like(x, device="cuda")
        exl3.had_r_128(x.cuda(), out, None if p is None else p.cuda(), None if q is None else q.cuda(), 1.5)
        ref = oracle.had_r_128(x.numpy(), None if p is None else p.numpy(), None if q is None else q.numpy(), 1.5)
        got = out.cpu().numpy()
        if dtype == torch.float16:
            d = np.abs(got.view(np.uint16).astype(np.int32) - ref.view(np.uint16).astype(np.int32))
            assert d.max() <= 1
        else:
            assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    # in place
    y = x.cuda()
    ref = oracle.had_r_128(x.numpy(), None, None, 1.0)
    exl3.had_r_128(y, y, None, None, 1.0)
    assert np.abs(y.cpu().numpy().astype(np.float64) - ref).max() <= 1e-3 * np.abs(ref).max()


def _linear_case(exl3, oracle, k, n, K, M, out_dtype, seed):
    S = synth()
    tr, suh, svh = S.linear(k, n, K, seed)
    x = S.activations(M, k, seed + 1)
    lin = exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), K, None, False, True, None)
    y = lin.run_alloc(x.cuda(), n, out_dtype == torch.float32)
    ref = oracle.exl3_linear(x.numpy(), tr.numpy(), suh.numpy(), svh.numpy(), K,
                             np.float32 if out_dtype == torch.float32 else np.float16)
    return y.cpu().numpy(), ref


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
def test_gemm_small_shapes(exl3, oracle, K, M):
    y, ref = _linear_case(exl3, oracle, 512, 384, K, M, torch.float32, 2000 + 10 * K + M)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M", [5, 9, 17])
def test_gemm_fp16_out_and_row_chunks(exl3, oracle, M):
    y, ref = _linear_case(exl3, oracle, 1024, 256, 3, M, torch.float16, 3000 + M)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M", [1, 4])
def test_gemm_c1_full_size(exl3, oracle, M):
    """Single dense linear 4096 -> 4096, K=4, fp16 output."""
    y, ref = _linear_case(exl3, oracle, 4096, 4096, 4, M, torch.float16, 1000)
    assert max_rel(y, ref) <= MAX_REL


def test_gemm_deterministic_and_bias(exl3):
    S = synth()
    tr, suh, svh = S.linear(2048, 1024, 3, 77)
    x = S.activations(3, 2048, 78).cuda()
    bias = torch.randn(1024).half().cuda()
    lin = exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), 3, None, False, True, None)
    y1 = lin.run_alloc(x, 1024, True)
    y2 = lin.run_alloc(x, 1024, True)
    assert torch.equal(y1, y2)
    lin_b = exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), 3, bias, False, True, None)
    y3 = lin_b.run_alloc(x, 1024, True)
    assert torch.allclose(y3, y1 + bias.float(), atol=1e-3)
    # run() with a preallocated fp16 output and a 3D input
    y4 = torch.empty(1, 3, 1024, dtype=torch.float16, device="cuda")
    lin.run(x.view(1, 3, 2048), y4)
    assert torch.allclose(y4.view(3, 1024).float(), y1, rtol=2e-3, atol=2e-3)


def test_gemm_one_row_tagged_exchange_across_shapes_and_graph_replays(exl3, oracle):
    """One-row calls exchange their split-K partials as tagged words that the last split clears: calls of different
    shapes back to back (other strip and split layouts over the same words), a one-row call between multi-row calls
    (which use the arrival counters), and replays of a captured one-row call each give the eager result bit for bit
    and match the oracle."""
    S = synth()
    shapes = [(4096, 4096, 4, 5100), (1024, 3072, 3, 5101), (5376, 2048, 2, 5102), (512, 384, 5, 5103)]
    cases = []
    for k, n, K, seed in shapes:
        tr, suh, svh = S.linear(k, n, K, seed)
        x = S.activations(3, k, seed + 1)
        lin = exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), K, None, False, True, None)
        ref = oracle.exl3_linear(x[:1].numpy(), tr.numpy(), suh.numpy(), svh.numpy(), K, np.float32)
        cases.append((lin, x.cuda(), n, ref))
    first = []
    for lin, x, n, ref in cases:
        y = lin.run_alloc(x[:1], n, True)
        assert max_rel(y.cpu().numpy(), ref) <= MAX_REL
        first.append(y)
    for _ in range(2):                                      # interleaved with three-row calls
        for (lin, x, n, _), y0 in zip(cases, first):
            lin.run_alloc(x, n, True)
            assert torch.equal(lin.run_alloc(x[:1], n, True), y0)
    lin, x, n, _ = cases[0]
    out = torch.empty(1, n, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lin.run(x[:1], out)                                 # sizes the workspace before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lin.run(x[:1], out)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first[0]), i
        c_lin, c_x, c_n, _ = cases[1 + i % 3]               # eager one-row work between the replays
        assert torch.equal(c_lin.run_alloc(c_x[:1], c_n, True), first[1 + i % 3])


# Rows >= 9 run on the MFMA path (row blocks of 16 / 32 / 64, k-split with partials summed by the last workgroup).
@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("M", [9, 24, 40, 64])
def test_gemm_mfma_rows_all_bitrates(exl3, oracle, K, M):
    y, ref = _linear_case(exl3, oracle, 512, 384, K, M, torch.float32, 4000 + 10 * K + M)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("jobs", [1, 64, 4096])
@pytest.mark.parametrize("M,out_dtype", [(16, torch.float16), (100, torch.float32), (130, torch.float16)])
def test_gemm_mfma_splits(exl3, oracle, monkeypatch, jobs, M, out_dtype):
    """Forced grid targets: one k-split (epilogue straight from the accumulators), and several (fp32 partials)."""
    monkeypatch.setenv("EXL3MI_LINEAR_JOBS", str(jobs))
    y, ref = _linear_case(exl3, oracle, 2048, 640, 3, M, out_dtype, 4500 + M + jobs)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M", [64, 300])
def test_gemm_mfma_c1_full_size(exl3, oracle, M):
    """4096 -> 4096, K=4 with a prefill-sized batch."""
    y, ref = _linear_case(exl3, oracle, 4096, 4096, 4, M, torch.float16, 1000 + M)
    assert max_rel(y, ref) <= MAX_REL


def test_gemm_mfma_strided_rows_and_determinism(exl3, oracle):
    """Through the C ABI: row strides wider than k / n on input and output (the columns past n untouched); repeated
    calls bit-identical; a 20-row call agrees with the same rows of the 70-row call."""
    from importlib import import_module
    L_ = import_module("b70-inference_amd._lib")
    S = synth()
    k, n, M, K = 1024, 512, 70, 2
    tr, suh, svh = S.linear(k, n, K, 4700)
    x = S.activations(M, k, 4701)
    xb = torch.zeros(M, k + 256, dtype=torch.float16)
    xb[:, :k] = x
    xb = xb.cuda()
    yb = torch.full((M, n + 128), 7.0, dtype=torch.float32, device="cuda")
    trc, suhc, svhc = tr.cuda(), suh.cuda(), svh.cuda()
    st = torch.cuda.current_stream().cuda_stream

    def run(rows, y):
        L_.check(L_.lib().exl3_gemm(L_.ptr(xb), k + 256, rows, k, L_.ptr(trc), n, K, L_.ptr(y), y.stride(0), 1,
                                    L_.ptr(suhc), None, L_.ptr(svhc), 2, st), "exl3_gemm")

    run(M, yb)
    y1 = yb[:, :n].clone()
    run(M, yb)
    torch.cuda.synchronize()
    assert torch.equal(y1, yb[:, :n])
    assert (yb[:, n:] == 7.0).all()
    ref = oracle.exl3_linear(x.numpy(), tr.numpy(), suh.numpy(), svh.numpy(), K, np.float32)
    assert max_rel(y1.cpu().numpy(), ref) <= MAX_REL
    y20 = torch.empty(20, n, dtype=torch.float32, device="cuda")
    run(20, y20)
    assert max_rel(y20.cpu().numpy(), ref[:20]) <= MAX_REL


@pytest.mark.parametrize("M", [1, 4, 9, 40, 100])
def test_linear_sharded_matches_per_shard_oracle(exl3, oracle, M):
    """Fused multi-projection linear (the XPU library's linear with suh[S, k] and shard_of_nb): three projections
    of widths 384 | 128 | 640 sharing the input, so 256-column blocks straddle shard boundaries; each column range
    equals its own projection's oracle output."""
    S_ = synth()
    k, widths, K = 1024, (384, 128, 640), 3
    shards = [S_.linear(k, n, K, 5000 + 10 * i) for i, n in enumerate(widths)]
    lins = [exl3.BC_LinearEXL3(tr.cuda(), su.cuda(), sv.cuda(), K, None, False, True, None) for tr, su, sv in shards]
    tr, suh, svh, sonb, bounds, Kf = exl3.fuse_linears(lins)
    x = S_.activations(M, k, 5100 + M)
    y = exl3.linear(x.cuda(), tr, suh, svh, sonb, bounds, Kf).float().cpu().numpy()
    for i, (t, su, sv) in enumerate(shards):
        ref = oracle.exl3_linear(x.numpy(), t.numpy(), su.numpy(), sv.numpy(), K, np.float16)
        assert max_rel(y[:, bounds[i]:bounds[i + 1]], ref) <= MAX_REL, i
    # fp32 output and the single-shard form agree with exl3_gemm
    y32 = torch.empty(M, sum(widths), dtype=torch.float32, device="cuda")
    exl3.linear(x.cuda(), tr, suh, svh, sonb, bounds, Kf, out=y32)
    assert max_rel(y32.cpu().numpy(), y) <= MAX_REL
    one = exl3.linear(x.cuda(), lins[2].trellis, lins[2].suh, lins[2].svh, None, [0, 640], K).float()
    assert torch.equal(one, lins[2].run_alloc(x.cuda(), 640, False).float())
