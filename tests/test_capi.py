"""The C-ABI library loads and exports every entry point include/exl3mi.h declares; host-side argument validation
returns the documented status codes (these calls return before any GPU work, so they run without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "exl3mi.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(exl3_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("exl3_last_error", "exl3_abi_version", "exl3_reconstruct", "exl3_had_r_128", "exl3_gemm"):
        assert s in syms


def test_library_exports_every_declared_symbol(exl3):
    L = exl3.lib()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    m = re.search(r"#define EXL3_ABI_VERSION (\d+)", open(HEADER).read())
    assert L.exl3_abi_version() == int(m.group(1))


def test_python_signatures_cover_header(exl3):
    from importlib import import_module
    sig = import_module("b70-inference_amd._lib").SIGNATURES
    assert set(declared_symbols()) <= set(sig), set(declared_symbols()) - set(sig)


def test_validation_errors(exl3):
    L = exl3.lib()
    vp = ctypes.c_void_p
    fake = vp(0x1000)
    # unsupported codebook and K -> EXL3_ERR_UNSUPPORTED, with a message
    assert L.exl3_gemm(fake, 256, 1, 256, fake, 256, 3, fake, 256, 0, fake, None, fake, 1, None) == 2
    assert b"codebook" in L.exl3_last_error()
    assert L.exl3_gemm(fake, 256, 1, 256, fake, 256, 9, fake, 256, 0, fake, None, fake, 2, None) == 2
    assert L.exl3_reconstruct(fake, 128, 128, 0, 2, 0, 128, fake, 128, None) == 2
    # shapes that are not multiples of 128 -> EXL3_ERR_INVALID
    assert L.exl3_gemm(fake, 200, 1, 200, fake, 256, 3, fake, 256, 0, fake, None, fake, 2, None) == 1
    assert L.exl3_reconstruct(fake, 128, 256, 3, 2, 64, 128, fake, 128, None) == 1
    assert L.exl3_had_r_128(fake, 100, fake, 100, 1, 100, 0, None, None, ctypes.c_float(1.0), None) == 1
    assert L.exl3_had_r_128(fake, 128, fake, 128, 1, 128, 5, None, None, ctypes.c_float(1.0), None) == 1
    # null pointers -> EXL3_ERR_INVALID
    assert L.exl3_gemm(None, 256, 1, 256, fake, 256, 3, fake, 256, 0, fake, None, fake, 2, None) == 1
    # m == 0 is a no-op
    assert L.exl3_gemm(fake, 256, 0, 256, fake, 256, 3, fake, 256, 0, fake, None, fake, 2, None) == 0
    # sharded linear: several shards need shard_of_nb; the shard count is bounded
    assert L.exl3_linear_sharded(fake, 256, 1, 256, fake, 256, 3, fake, 256, 0, fake, 2, None, fake, 2, None) == 1
    assert L.exl3_linear_sharded(fake, 256, 1, 256, fake, 256, 3, fake, 256, 0, fake, 0, None, fake, 2, None) == 1
    assert L.exl3_linear_sharded(fake, 256, 0, 256, fake, 256, 3, fake, 256, 0, fake, 2, fake, fake, 2, None) == 0
    # routers: scoring and flags are checked, sizes as the softmax router
    assert L.exl3_route_topk(fake, 64, 1, 64, None, 4, 7, 1, ctypes.c_float(1.0), fake, fake, None) == 2
    assert L.exl3_route_topk(fake, 64, 1, 64, None, 4, 1, 8, ctypes.c_float(1.0), fake, fake, None) == 1
    assert L.exl3_route_topk(fake, 64, 1, 64, None, 40, 1, 1, ctypes.c_float(1.0), fake, fake, None) == 1
    assert L.exl3_router_logits(fake, 200, 1, 200, fake, 64, 64, 0, 0, fake, 64, None) == 1
    assert L.exl3_router_logits(fake, 256, 1, 256, fake, 60, 60, 0, 0, fake, 60, None) == 1
    assert L.exl3_router_logits(fake, 256, 1, 256, fake, 64, 64, 2, 0, fake, 64, None) == 1


def test_python_errors_match_reference(exl3):
    import torch
    tr = torch.zeros(16, 16, 48, dtype=torch.int16)
    s = torch.ones(256, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        exl3.BC_LinearEXL3(tr, s, s, 3, None, True, False, None)      # mcg codebook
    with pytest.raises(NotImplementedError):
        exl3.BC_LinearEXL3(torch.zeros(16, 16, 40, dtype=torch.int16), s, s, 2.5, None, False, True, None)
