"""ctypes binding of libexl3mi.so (the HIP kernels and their C ABI, declared in include/exl3mi.h).

The library is built in-tree (csrc/Makefile, driven by __graft_entry__.build()). There is no fallback: if the shared
library is missing, every op raises, so a GPU run can never silently take a non-HIP path.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EXL3MI_LIB") or os.path.join(HERE, "libexl3mi.so")

EXL3_OK, EXL3_ERR_INVALID, EXL3_ERR_UNSUPPORTED, EXL3_ERR_HIP = 0, 1, 2, 3
EXL3_F16, EXL3_F32 = 0, 1
EXL3_WORDS_PLANAR4, EXL3_WORDS_TILE_ORDER = 0, 1
ACT_SILU, ACT_GELU_TANH = 0, 1

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# name -> argtypes; every entry point returns int (exl3_status) unless listed in _RESTYPE
SIGNATURES = {
    "exl3_last_error": [],
    "exl3_abi_version": [],
    "exl3_reserve_workspace": [_i64, _i64],
    "exl3_device_status": [_vp],
    "exl3_release_workspace": [],
    "exl3_profile_enable": [_i32],
    "exl3_profile_read": [ctypes.c_char_p, _i64],
    "exl3_reconstruct": [_vp, _i64, _i64, _i32, _i32, _i64, _i64, _vp, _i64, _vp],
    "exl3_reconstruct_had_slice": [_vp, _i64, _i64, _i32, _i32, _vp, _vp, _i64, _i64, _vp, _i64, _vp],
    "exl3_had_r_128": [_vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _vp, _f32, _vp],
    "exl3_gemm": [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp, _i32, _vp],
    "exl3_gemm_noalloc": [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp],
    "exl3_linear_sharded": [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _vp, _vp, _i32, _vp],
    "exl3_mgemm": [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _i64, _i64, _i64, _vp,
                   _i32, _vp],
    "exl3_act_mul": [_vp, _vp, _vp, _i64, _i32, _i32, _f32, _vp],
    "exl3_route_adjusted": [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _f32, _vp, _vp, _vp],
    "exl3_route_block": [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _f32, _f32, _vp, _vp, _vp],
    "exl3_moe_forward": [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _f32,
                         _i64, _vp, _i64, _i32, _vp],
    "exl3_moe_forward_blobs": [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _i32, _i32, _f32, _vp, _i64,
                               _i32, _i32, _vp],
    "exl3_blob_unplanarize": [_vp, _i64, _i64, _i64, _i32, _vp],
    "exl3_moe_forward_logits": [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _i32,
                                _i32, _i32, _f32, _i64, _vp, _vp, _vp, _vp, _i64, _i32, _vp],
    "exl3_moe_align": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp],
    "exl3_route_softmax_topk": [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp],
    "exl3_route_topk": [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _f32, _vp, _vp, _vp],
    "exl3_router_logits": [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp],
}
_RESTYPE = {"exl3_last_error": ctypes.c_char_p}

_lib = None


class Exl3Error(RuntimeError):
    pass


def lib():
    """Load the shared library (once). Raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Exl3Error(f"exl3mi: {LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        _lib = L
    return _lib


def check(rc: int, what: str = ""):
    """Map a C status to the exception the reference raises for the same condition."""
    if rc == EXL3_OK:
        return
    msg = lib().exl3_last_error().decode(errors="replace")
    if rc == EXL3_ERR_UNSUPPORTED:
        raise NotImplementedError(msg or what)
    raise Exl3Error(msg or f"{what}: status {rc}")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The caller's current stream on t's device (launches are asynchronous on it, as in the reference)."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def profile_enable(on: bool = True, repeat: int = 1):
    """Event-time every library launch on its stream; repeat > 1 runs each launch that many times per event pair."""
    check(lib().exl3_profile_enable(max(1, int(repeat)) if on else 0), "exl3_profile_enable")


def profile_read() -> dict:
    """{kernel name: (launches, average microseconds)} since the last profile_enable (synchronises)."""
    buf = ctypes.create_string_buffer(1 << 16)
    check(lib().exl3_profile_read(buf, len(buf)), "exl3_profile_read")
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, avg = line.rsplit(" ", 2)
        out[name] = (int(cnt), float(avg))
    return out


def device_status() -> int:
    """The current device's status word: non-zero after a fused MoE layer or split-K GEMV launch gave up waiting (read
    on the host, no synchronisation; the next library call on the device reports and clears it)."""
    v = ctypes.c_int(0)
    check(lib().exl3_device_status(ctypes.byref(v)), "exl3_device_status")
    return v.value


def reserve_workspace(nbytes: int, ncounters: int = 0):
    """Pre-size this device's workspace (e.g. before HIP graph capture; growth is refused while capturing)."""
    check(lib().exl3_reserve_workspace(int(nbytes), int(ncounters)), "exl3_reserve_workspace")


def release_workspace():
    """Free outgrown workspace buffers (synchronises; no graph captured before may be replayed afterwards)."""
    check(lib().exl3_release_workspace(), "exl3_release_workspace")


def require_device(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise Exl3Error(f"exl3mi: tensors must be on a GPU, got {t.device}")
