"""exl3_gemm_noalloc (the decode GEMV with its scratch in a fixed per-device array) against exl3_gemm, called through
the C ABI: bit-identical outputs on two calls in a row, the second smaller, plus its size limits."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
synth = importlib.import_module("b70-inference_amd.synth")


def _case(k, n, K, m, seed):
    tr, suh, svh = synth.linear(k, n, K, seed)
    x = synth.activations(m, k, seed + 1)
    return tr.cuda(), suh.cuda(), svh.cuda(), x.cuda()


def _call(L, name, tr, suh, svh, x, out):
    k, n, m = x.shape[1], out.shape[1], x.shape[0]
    K = tr.shape[-1] // 16
    dt = 1 if out.dtype == torch.float32 else 0
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = ctypes.c_void_p
    if name == "exl3_gemm":
        rc = L.exl3_gemm(vp(x.data_ptr()), k, m, k, vp(tr.data_ptr()), n, K, vp(out.data_ptr()), n, dt,
                         vp(suh.data_ptr()), None, vp(svh.data_ptr()), 2, st)
    else:
        rc = L.exl3_gemm_noalloc(vp(x.data_ptr()), k, m, k, vp(tr.data_ptr()), n, K, vp(out.data_ptr()), n, dt,
                                 vp(suh.data_ptr()), vp(svh.data_ptr()), 2, st)
    assert rc == 0, L.exl3_last_error()


def test_noalloc_matches_exl3_gemm_two_calls(exl3, oracle):
    L = exl3.lib()
    # a C2-sized projection (5376 -> 21504, K = 4, 4 rows, fp32 out), then a smaller one (1024 -> 2048, K = 3, 1 row,
    # fp16 out): the second call reuses the array the first one left
    cases = ((5376, 21504, 4, 4, torch.float32, 7100), (1024, 2048, 3, 1, torch.float16, 7200))
    for (k, n, K, m, dtype, seed) in cases:
        print(f"no-alloc test: k={k} n={n} K={K} m={m} {dtype}", flush=True)
        tr, suh, svh, x = _case(k, n, K, m, seed)
        ref = torch.full((m, n), float("nan"), dtype=dtype, device="cuda")
        got = torch.full((m, n), float("nan"), dtype=dtype, device="cuda")
        _call(L, "exl3_gemm", tr, suh, svh, x, ref)
        _call(L, "exl3_gemm_noalloc", tr, suh, svh, x, got)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        if k == 1024:
            r = oracle.exl3_linear(x.cpu().numpy(), tr.cpu().numpy(), suh.cpu().numpy(), svh.cpu().numpy(), K,
                                   np.float16).astype(np.float64)
            assert np.abs(got.cpu().numpy() - r).max() / np.abs(r).max() <= 2e-3


def test_noalloc_rejects_shapes_beyond_its_scratch(exl3):
    L = exl3.lib()
    fake = ctypes.c_void_p(0x1000)
    st = ctypes.c_void_p(0)
    # 9 rows: beyond the decode GEMV
    assert L.exl3_gemm_noalloc(fake, 256, 9, 256, fake, 256, 3, fake, 256, 0, fake, fake, 2, st) == 1
    assert b"at most 8" in L.exl3_last_error()
    # more columns than the fixed counters cover
    n = 16384 * 128 + 128
    assert L.exl3_gemm_noalloc(fake, 256, 1, 256, fake, n, 1, fake, n, 0, fake, fake, 2, st) == 1
    # partials beyond 16 MiB: 8192 strips x 1 split x 4 KiB = 32 MiB
    n = 8192 * 128
    assert L.exl3_gemm_noalloc(fake, 128, 1, 128, fake, n, 1, fake, n, 0, fake, fake, 2, st) == 1
    assert b"partials" in L.exl3_last_error()
