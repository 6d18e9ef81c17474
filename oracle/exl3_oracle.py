"""NumPy restatement of the EXL3 (exllamav3 trellis, mul1 codebook) linear and MoE-layer semantics.

TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU baseline. The product never imports it.

Sources restated (paths relative to the reference root):
  * bitstream + window     glm/docs/ext-op-inventory.md:717-725, 746-757; glm/xpu/csrc/exl3_esimd.h:4-14, 117-149;
                           dsv41/xpu/dsv_xpu/exl3_tri.py:22-35
  * mul1 codebook          glm/xpu/csrc/exl3_esimd.h:40-68; ext-op-inventory.md:559-571, 738-743
  * position -> (row,col)  glm/xpu/csrc/exl3_esimd.h:7-8; ext-op-inventory.md:727-733
  * reconstruct            glm/xpu/csrc/exl3_ops.sycl:539-555; ext-op-inventory.md:597-612, 758-760
  * had_r_128              ext-op-inventory.md:576-595; glm/xpu/glm_xpu/ops.py:118-142
  * linear                 ext-op-inventory.md:512-535, 707-712, 762-773
  * multi-matrix linear    ext-op-inventory.md:664-685 (exl3_mgemm: slots, indices, min/max filter, weighted sum)
  * expert math / MoE      ext-op-inventory.md:923-942; glm/xpu/csrc/exl3_moe.n128.sycl:253-271, 370-379, 405-408;
                           dsv41/xpu/dsv_xpu/moe.py:967-994
  * activations            ext-op-inventory.md:944-956 (SiLU, act_limit clamp); GELU-tanh = torch gelu(approximate='tanh')
  * routing                trellis-serve.patch:395-441 (softmax -> top-k -> renormalise, +1e-20); sigmoid + bias,
                           glm/xpu/glm_xpu/ops.py:177-193; sqrt-softplus, dsv41/xpu/csrc/dsv_moe_glue.sycl:155-193
  * router logits          glm/xpu/glm_xpu/ops.py:183-184 (x @ gate[:, :E]); dsv_moe_glue.sycl:442-470 (x @ W^T)
  * expert blob            glm/xpu/exl3xpu/moe_offload.py:68-94 (planar4, pack_expert); glm/xpu/pack_store.py:35-60
                           (blob_perm); glm/xpu/csrc/exl3_moe.n128.sycl:56-68 (Geom byte offsets)
  * align / pair lists     glm/xpu/csrc/exl3_moe.n128.sycl:691-734

How each function is pinned (tests/test_oracle.py, tests/test_blob.py): codebook against six textual statements
over all 65536 states; windows / reconstruct against the brute-force C ring decoder (oracle/trellis_bruteforce.c)
for K = 1..8; permutation by three statements and bijectivity; Hadamard by orthogonality, basis rows and the dense
+-1 matmul; linear and MoE by the dense-weight form built the other way round; activations against
torch.nn.functional gelu(approximate='tanh') / silu in float64 (with the clamp form); routing by hand-built ties and
invariants; PLANAR4 against an element-by-element loop of the reference's stated index map. No function is
"parity unpinned"; what stays unpinned is the un-vendored exllamav3 / trellis-serve code at the boundary (their
testlib and packer), for which the agreeing statements above stand in.

Every floating-point reduction here runs in float64 unless a caller asks for float32 (`acc`), so the oracle is at
least as accurate as the fp32-accumulated reference. Rounding points that the reference fixes (fp16 x*suh, fp16
transformed activations, fp16 gate/up/act) are reproduced exactly.
"""
from __future__ import annotations

import math

import numpy as np

MUL1 = 0x83DCD12D
K_INV = 0.00676727294921875      # fp16 bit pattern 0x1EEE
K_BIAS = -10.3828125             # fp16 bit pattern 0xC931
RSQRT128 = 1.0 / math.sqrt(128.0)

# ------------------------------------------------------------------------------------------------ codebook


def mul1_values(states: np.ndarray) -> np.ndarray:
    """mul1 codebook on 16-bit states -> float16. x = st * 0x83DCD12D mod 2^32, s = byte sum of x,
    w = fp16((1024 + s) * K_INV + K_BIAS) with one rounding (exl3_esimd.h:46-68, inventory:559-571).
    (1024 + s) * K_INV is exact in float64 and in float32, so the single rounding is the cast to float16."""
    st = np.asarray(states, dtype=np.uint64) & 0xFFFF
    x = (st * MUL1) & 0xFFFFFFFF
    s = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + ((x >> 24) & 0xFF)
    v = (1024.0 + s.astype(np.float64)) * K_INV + K_BIAS
    return v.astype(np.float16)


_LUT = None


def mul1_lut() -> np.ndarray:
    """[65536] float16: the codebook value of every 16-bit state."""
    global _LUT
    if _LUT is None:
        _LUT = mul1_values(np.arange(65536, dtype=np.uint64))
        _LUT.setflags(write=False)
    return _LUT


# ------------------------------------------------------------------------------------------------ tile layout


def pos_row_col():
    """Position t (0..255) of the tile stream -> (row, col) of the 16x16 tile; row is the input (k) index, col the
    output (n) index (exl3_esimd.h:7-8, inventory:727-733)."""
    t = np.arange(256)
    row = 8 * ((t >> 1) & 1) + 2 * ((t >> 3) & 3) + (t & 1)
    col = (t >> 5) + 8 * ((t >> 2) & 1)
    return row, col


def tile_states(words: np.ndarray, K: int) -> np.ndarray:
    """words [..., 8K] uint32 (little-endian int16 pairs) -> [..., 256] 16-bit states. Position t's state is the
    window of stream bits [(t+1)K - 16, (t+1)K), MSB-first, circular within the tile (inventory:746-757)."""
    assert 1 <= K <= 8
    w = np.asarray(words, dtype=np.uint64)
    assert w.shape[-1] == 8 * K
    t = np.arange(256)
    e = (t + 1) * K
    ih = (e - 1) // 32
    sh = (32 * (ih + 1) - e).astype(np.uint64)
    il = (ih - 1) % (8 * K)
    st = (((w[..., il] << np.uint64(32)) | w[..., ih]) >> sh) & np.uint64(0xFFFF)
    return st.astype(np.uint16)


def trellis_words(trellis: np.ndarray) -> np.ndarray:
    """int16 [tk, tn, 16K] -> uint32 [tk, tn, 8K] (word i = u16[2i] | u16[2i+1] << 16)."""
    tr = np.ascontiguousarray(trellis)
    assert tr.dtype == np.int16 and tr.shape[-1] % 16 == 0
    return tr.view(np.uint32)


def decode_tiles(words: np.ndarray, K: int) -> np.ndarray:
    """uint32 [..., 8K] -> float16 [..., 16, 16] (tile[row, col])."""
    vals = mul1_lut()[tile_states(words, K)]
    row, col = pos_row_col()
    tiles = np.empty(vals.shape[:-1] + (16, 16), dtype=np.float16)
    tiles[..., row, col] = vals
    return tiles


def reconstruct(trellis: np.ndarray, K: int, n0: int = 0, n_slice: int | None = None) -> np.ndarray:
    """W_hat[:, n0 : n0 + n_slice] as float16 [k, n_slice], Hadamard domain, no sign vectors
    (exl3_ops.sycl:539-555, inventory:597-612, 758-760)."""
    tk, tn, w = trellis.shape
    assert w == 16 * K
    if n_slice is None:
        n_slice = tn * 16 - n0
    assert n0 % 16 == 0 and n_slice % 16 == 0 and n0 + n_slice <= tn * 16
    words = trellis_words(trellis)[:, n0 // 16:(n0 + n_slice) // 16]
    tiles = decode_tiles(words, K)                                        # [tk, tn', 16, 16]
    return tiles.transpose(0, 2, 1, 3).reshape(tk * 16, n_slice)


# Fast C statement of the same decode (oracle/trellis_fast.c, built into oracle/_build/libexl3_oracle.so), pinned bit
# for bit against reconstruct / reconstruct_mixed and the brute-force decoder; Proj uses it for large matrices.
_FAST = None


def _fast_lib():
    global _FAST
    if _FAST is None:
        import ctypes
        import os
        import subprocess
        here = os.path.dirname(os.path.abspath(__file__))
        path = os.path.join(here, "_build", "libexl3_oracle.so")
        if not os.path.exists(path):
            subprocess.run(["make", "-C", here], check=True, capture_output=True)
        L = ctypes.CDLL(path)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.exl3_fast_reconstruct.argtypes = [vp, i64, i64, i32, i64, i64, vp, i32]
        L.exl3_fast_reconstruct_mixed.argtypes = [vp, vp, vp, i64, i64, vp, i32]
        L.exl3_fast_matmul.argtypes = [vp, i64, i64, i32, vp, i64, vp, i32]
        L.exl3_fast_matmul_mixed.argtypes = [vp, vp, vp, i64, i64, vp, i64, vp, i32]
        _FAST = L
    return _FAST


def _threads() -> int:
    """Every core this process may run on, capped by OMP_NUM_THREADS when that is set (a host's CPU share)."""
    import os
    n = len(os.sched_getaffinity(0))
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        cap = 0
    return max(1, min(n, cap) if cap > 0 else n)


def reconstruct_fast(trellis: np.ndarray, K: int, n0: int = 0, n_slice: int | None = None) -> np.ndarray:
    """reconstruct() through the C decoder, multithreaded."""
    tr = np.ascontiguousarray(trellis, dtype=np.int16)
    tk, tn, w = tr.shape
    assert w == 16 * K
    if n_slice is None:
        n_slice = tn * 16 - n0
    assert n0 % 16 == 0 and n_slice % 16 == 0 and n0 + n_slice <= tn * 16
    out = np.empty((tk * 16, n_slice), dtype=np.uint16)
    rc = _fast_lib().exl3_fast_reconstruct(tr.ctypes.data, tk, tn, K, n0 // 16, n_slice // 16, out.ctypes.data,
                                           _threads())
    assert rc == 0
    return out.view(np.float16)


def reconstruct_mixed_fast(words: np.ndarray, kmap: np.ndarray, woff: np.ndarray, k: int, n: int) -> np.ndarray:
    """reconstruct_mixed() through the C decoder, multithreaded."""
    w = np.ascontiguousarray(words).view(np.uint32)
    km = np.ascontiguousarray(kmap, dtype=np.uint8).reshape(-1)
    wo = np.ascontiguousarray(woff, dtype=np.int64).reshape(-1)
    tk, tn = k // 16, n // 16
    assert km.size == tk * tn and wo.size == tk * tn + 1 and int(wo[-1]) <= w.size
    out = np.empty((k, n), dtype=np.uint16)
    rc = _fast_lib().exl3_fast_reconstruct_mixed(w.ctypes.data, km.ctypes.data, wo.ctypes.data, tk, tn,
                                                 out.ctypes.data, _threads())
    assert rc == 0
    return out.view(np.float16)


def matmul_fast(xh: np.ndarray, trellis=None, K=None, words=None, kmap=None, woff=None) -> np.ndarray:
    """xh @ W_hat in float64 (= linear_acc(xh, reconstruct(...))) through the C decoder, without materialising W_hat:
    uniform K (`trellis`, `K`) or per-tile K (`words`, `kmap`, `woff`). xh [m, k] -> float64 [m, n]."""
    x = np.ascontiguousarray(xh, dtype=np.float64)
    m = x.shape[0]
    if trellis is not None:
        tr = np.ascontiguousarray(trellis, dtype=np.int16)
        tk, tn, w = tr.shape
        assert w == 16 * K and x.shape[1] == tk * 16
        y = np.empty((m, tn * 16), dtype=np.float64)
        assert _fast_lib().exl3_fast_matmul(tr.ctypes.data, tk, tn, K, x.ctypes.data, m, y.ctypes.data,
                                            _threads()) == 0
        return y
    wd = np.ascontiguousarray(words).view(np.uint32)
    km = np.ascontiguousarray(kmap, dtype=np.uint8).reshape(-1)
    wo = np.ascontiguousarray(woff, dtype=np.int64).reshape(-1)
    tk = x.shape[1] // 16
    tn = km.size // tk
    assert km.size == tk * tn and wo.size == tk * tn + 1 and int(wo[-1]) <= wd.size
    y = np.empty((m, tn * 16), dtype=np.float64)
    assert _fast_lib().exl3_fast_matmul_mixed(wd.ctypes.data, km.ctypes.data, wo.ctypes.data, tk, tn, x.ctypes.data,
                                              m, y.ctypes.data, _threads()) == 0
    return y


def reconstruct_mixed(words: np.ndarray, kmap: np.ndarray, woff: np.ndarray, k: int, n: int) -> np.ndarray:
    """Per-tile K: tile i (row-major over [k/16, n/16]) is stored at words[woff[i] : woff[i] + 8 kmap[i]]."""
    tk, tn = k // 16, n // 16
    kmap = np.asarray(kmap).reshape(-1)
    woff = np.asarray(woff, dtype=np.int64).reshape(-1)
    assert kmap.size == tk * tn and woff.size == tk * tn + 1
    tiles = np.empty((tk * tn, 16, 16), dtype=np.float16)
    for K in np.unique(kmap):
        idx = np.nonzero(kmap == K)[0]
        gather = woff[idx][:, None] + np.arange(8 * int(K))[None, :]
        tiles[idx] = decode_tiles(words[gather], int(K))
    return tiles.reshape(tk, tn, 16, 16).transpose(0, 2, 1, 3).reshape(k, n)


# ------------------------------------------------------------------------------------------------ Hadamard

_H = None


def sylvester128() -> np.ndarray:
    """Natural-order Sylvester H128, entries +-1, H[i, j] = (-1)^popcount(i & j) (inventory:514-516)."""
    global _H
    if _H is None:
        h = np.ones((1, 1))
        while h.shape[0] < 128:
            h = np.block([[h, h], [h, -h]])
        _H = h
        _H.setflags(write=False)
    return _H


def had_blocks(v: np.ndarray) -> np.ndarray:
    """Blockwise unnormalised H128 along the last axis, float64."""
    s = v.shape
    return (np.asarray(v, dtype=np.float64).reshape(-1, 128) @ sylvester128()).reshape(s)


def had_r_128(x: np.ndarray, pre: np.ndarray | None = None, post: np.ndarray | None = None, scale: float = 1.0,
              out_dtype=None) -> np.ndarray:
    """exllamav3 had_r_128 (inventory:576-595). fp16 path: x*pre rounded to fp16, butterfly exact, *scale/sqrt(128),
    rounded to fp16, then *post rounded to fp16. fp32 path: no intermediate roundings. If both pre and post are given
    only pre is applied (the reference's if/else chain)."""
    if out_dtype is None:
        out_dtype = x.dtype
    r = scale * RSQRT128
    if x.dtype == np.float16:
        v = x if pre is None else (x.astype(np.float32) * pre.astype(np.float32)).astype(np.float16)
        y = (had_blocks(v) * r).astype(np.float16)
        if pre is None and post is not None:
            y = (y.astype(np.float32) * post.astype(np.float32)).astype(np.float16)
        return y.astype(out_dtype)
    v = x.astype(np.float64) if pre is None else x.astype(np.float64) * pre.astype(np.float64)
    y = had_blocks(v) * r
    if pre is None and post is not None:
        y = y * post.astype(np.float64)
    return y.astype(out_dtype)


def had_in(x: np.ndarray, suh: np.ndarray) -> np.ndarray:
    """Input transform: fp16( H128(fp16(x * suh)) / sqrt(128) ) (inventory:523-525, exl3_esimd.h:300)."""
    return had_r_128(x.astype(np.float16), pre=suh.astype(np.float16))


# ------------------------------------------------------------------------------------------------ linear


def linear_acc(xh: np.ndarray, W: np.ndarray, acc=np.float64) -> np.ndarray:
    return xh.astype(acc) @ W.astype(acc)


def had_out(acc: np.ndarray, svh: np.ndarray, out_dtype) -> np.ndarray:
    """Output transform: H128(acc) / sqrt(128) * svh; fp16 outputs round once at the end (XPU form,
    exl3_esimd.h:317-338; the CUDA fp16 form rounds before *svh, within 1 ulp)."""
    y = had_blocks(acc) * RSQRT128 * svh.astype(np.float64)
    return y.astype(out_dtype)


def exl3_linear(x: np.ndarray, trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int,
                out_dtype=np.float32, acc=np.float64, W: np.ndarray | None = None) -> np.ndarray:
    """y = Hn( Hk(x * suh) @ W_hat ) * svh with the reference rounding points (inventory:512-535)."""
    x2 = x.reshape(-1, x.shape[-1])
    xh = had_in(x2, suh)
    if W is None:
        W = reconstruct(trellis, K)
    y = had_out(linear_acc(xh, W, acc), svh, out_dtype)
    return y.reshape(x.shape[:-1] + (y.shape[-1],))


def mgemm_matrix(indices, j: int, nmat: int, min_index: int = -1, max_index: int = -1) -> int:
    """Matrix of slot j of exl3_mgemm: indices[j] (j without indices), filtered to [min_index, max_index) and rebased
    when min_index >= 0; -1 (slot skipped) for a negative or out-of-range result (inventory:677-682)."""
    q = int(indices[j]) if indices is not None else j
    if min_index >= 0:
        q = q - min_index if min_index <= q < max_index else -1
    return q if 0 <= q < nmat else -1


def mgemm(A: np.ndarray, mats, K: int, indices=None, weights=None, num_tokens: int = 1, min_index: int = -1,
          max_index: int = -1, slots: int | None = None, out_dtype=np.float32, C=None):
    """exllamav3 exl3_mgemm (inventory:664-685). A [a_batches, m, k]; mats = [(trellis, suh, svh)]; slot j runs
    matrix mgemm_matrix(j) on A batch 0 / j / j // (slots // num_tokens) (a_batches 1 / slots / num_tokens).
    Without weights returns C [slots, m, n] (skipped slots keep C's rows: C given, else zeros); with weights
    C[t] = sum over token t's slots in order of weights[j] * Y_j, in float64 then out_dtype."""
    A = np.asarray(A)
    a_batches = A.shape[0]
    if slots is None:
        slots = len(indices) if indices is not None else len(mats)
    per_tok = slots // num_tokens if num_tokens else 0
    n = mats[0][0].shape[1] * 16

    def a_of(j):
        if a_batches == 1:
            return A[0]
        return A[j] if a_batches == slots else A[j // per_tok]

    ys = []
    for j in range(slots):
        q = mgemm_matrix(indices, j, len(mats), min_index, max_index)
        if q < 0:
            ys.append(None)
            continue
        tr, suh, svh = mats[q]
        y = exl3_linear(a_of(j), tr, suh, svh, K, np.float64 if weights is not None else out_dtype)
        ys.append(y)
    if weights is None:
        out = np.array(C, copy=True) if C is not None else np.zeros((slots, A.shape[1], n), out_dtype)
        for j, y in enumerate(ys):
            if y is not None:
                out[j] = y
        return out
    w = np.asarray(weights, dtype=np.float16).astype(np.float64)
    out = np.zeros((num_tokens, A.shape[1], n), np.float64)
    for t in range(num_tokens):
        for i in range(per_tok):
            j = t * per_tok + i
            if ys[j] is not None:
                out[t] += w[j] * ys[j]
    return out.astype(out_dtype)


def dense_weight(trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int) -> np.ndarray:
    """Original-basis weight W = diag(suh) Hblk W_hat Hblk diag(svh), float64 (inventory:707-712)."""
    Wh = reconstruct(trellis, K).astype(np.float64)
    k, n = Wh.shape
    Hb = sylvester128() * RSQRT128
    # Hblk W_hat: transform every 128-block of rows; W_hat Hblk: every 128-block of columns
    t = (Hb @ Wh.reshape(k // 128, 128, n)).reshape(k, n)
    t = (t.reshape(k, n // 128, 128) @ Hb).reshape(k, n)
    return suh.astype(np.float64)[:, None] * t * svh.astype(np.float64)[None, :]


# ------------------------------------------------------------------------------------------------ activations

ACT_SILU, ACT_GELU_TANH = 0, 1


def act_mul(g: np.ndarray, u: np.ndarray, act: int, limit: float = 0.0) -> np.ndarray:
    """Gated activation in float64, rounded to fp16 by the caller.
    SiLU: a = min(silu(g), L) * clamp(u, -L, L), L = 0 disables the clamp (inventory:944-956).
    GELU-tanh: a = 0.5 g (1 + tanh(sqrt(2/pi)(g + 0.044715 g^3))) * u (inventory:311, 892)."""
    g = g.astype(np.float64)
    u = u.astype(np.float64)
    if act == ACT_SILU:
        with np.errstate(over="ignore"):  # exp(-g) = inf for g < -709 gives the exact limit s = -0.0
            s = g / (1.0 + np.exp(-g))
        if limit:
            s = np.minimum(s, limit)
            u = np.clip(u, -limit, limit)
        return s * u
    if act == ACT_GELU_TANH:
        c = math.sqrt(2.0 / math.pi)
        return 0.5 * g * (1.0 + np.tanh(c * (g + 0.044715 * g ** 3))) * u
    raise ValueError(act)


# ------------------------------------------------------------------------------------------------ MLP / MoE


class Proj:
    """One EXL3 projection. Uniform K (`trellis` int16 [k/16, n/16, 16K]) or per-tile K (`words`, `kmap`, `woff`)."""

    def __init__(self, suh, svh, trellis=None, K=None, words=None, kmap=None, woff=None):
        self.suh, self.svh = suh, svh
        self.trellis, self.K = trellis, K
        self.words, self.kmap, self.woff = words, kmap, woff
        self.k, self.n = suh.shape[0], svh.shape[0]
        self._W = None

    def W(self) -> np.ndarray:
        """W_hat fp16 [k, n]: the NumPy statement for small matrices, the (pinned, identical) C decoder from 2^20
        weights on."""
        if self._W is None:
            fast = self.k * self.n >= (1 << 20)
            if self.trellis is not None:
                self._W = (reconstruct_fast if fast else reconstruct)(self.trellis, self.K)
            else:
                self._W = (reconstruct_mixed_fast if fast else reconstruct_mixed)(self.words, self.kmap, self.woff,
                                                                                  self.k, self.n)
        return self._W

    def drop(self):
        self._W = None

    def __call__(self, x, out_dtype, acc=np.float64):
        xh = had_in(x.reshape(-1, self.k), self.suh)
        if acc == np.float64 and self._W is None and self.k * self.n >= (1 << 20):
            # large matrices in float64: decode and multiply in C (same sums, W_hat never materialised)
            if self.trellis is not None:
                y = matmul_fast(xh, trellis=self.trellis, K=self.K)
            else:
                y = matmul_fast(xh, words=self.words, kmap=self.kmap, woff=self.woff)
            return had_out(y, self.svh, out_dtype)
        return had_out(linear_acc(xh, self.W(), acc), self.svh, out_dtype)


def gated_mlp(x: np.ndarray, gate: Proj, up: Proj, down: Proj, act: int, limit: float = 0.0,
              acc=np.float64) -> np.ndarray:
    """g, u = gate(x), up(x) (fp16); a = fp16(act(g, u)); d = down(a) (fp32) (inventory:923-942, 1172-1187)."""
    g = gate(x, np.float16, acc)
    u = up(x, np.float16, acc)
    a = act_mul(g, u, act, limit).astype(np.float16)
    return down(a, np.float32, acc)


def moe_layer(x: np.ndarray, experts, ids: np.ndarray, w: np.ndarray, act: int = ACT_SILU, limit: float = 0.0,
              shared=None, acc=np.float64, drop_weights: bool = False) -> np.ndarray:
    """out[t] = sum_{j in slot order} w[t, j] * expert_{ids[t, j]}(x[t]) (fp32 sum) + shared(x[t]).
    `experts[e]` is a (gate, up, down) tuple of Proj. Slots with ids < 0 are inactive. Output float32 [M, H]."""
    M, H = x.shape
    y = np.zeros((M, ids.shape[1], H), dtype=np.float64)
    for e in np.unique(ids[ids >= 0]):
        rows, slots = np.nonzero(ids == e)
        d = gated_mlp(x[rows], *experts[int(e)], act, limit, acc)
        y[rows, slots] = d.astype(np.float64) * w[rows, slots].astype(np.float64)[:, None]
        if drop_weights:
            for p in experts[int(e)]:
                p.drop()
    out = np.zeros((M, H), dtype=np.float32)
    for j in range(ids.shape[1]):                       # fixed slot order, fp32 sum
        out += y[:, j].astype(np.float32)
    if shared is not None:
        out += gated_mlp(x, *shared, act, limit, acc)
    return out


# ------------------------------------------------------------------------------------------------ routing


def topk_lowest_index(key: np.ndarray, k: int) -> np.ndarray:
    """Top-k indices by descending key; exact ties go to the lower expert index."""
    order = np.argsort(-key, axis=-1, kind="stable")
    return order[..., :k]


def route_softmax_topk(logits: np.ndarray, k: int, bias: np.ndarray | None = None):
    """softmax over (logits + bias) -> top-k -> renormalise with +1e-20 (trellis-serve.patch:395-441).
    Returns ids int32 [M, k] (descending probability) and w float32 [M, k]."""
    z = logits.astype(np.float32)
    if bias is not None:
        z = z + bias.astype(np.float32)[None, :]
    z64 = z.astype(np.float64)
    p = np.exp(z64 - z64.max(-1, keepdims=True))
    p = p / p.sum(-1, keepdims=True)
    ids = topk_lowest_index(z, k)
    pw = np.take_along_axis(p, ids, -1)
    w = pw / (pw.sum(-1, keepdims=True) + 1e-20)
    return ids.astype(np.int32), w.astype(np.float32)


SCORES = ("softmax", "sigmoid", "sqrt_softplus")


def route_topk(logits: np.ndarray, k: int, bias: np.ndarray | None = None, score: str = "softmax",
               renorm: bool = True, scaling: float = 1.0, bias_select_only: bool = False,
               mul: np.ndarray | None = None, res: np.ndarray | None = None):
    """Top-k routing with a scoring function; ranking values in float32 (as the kernel ranks), weights in float64.
      softmax        rank by f + b; weights from softmax(f + b), or softmax(f) when the bias only selects
                     (trellis-serve.patch:395-441, its `cold` term)
      sigmoid        s = sigmoid(f); rank by s + b, by f without a bias; weights from s (glm/xpu/glm_xpu/ops.py:186-191)
      sqrt_softplus  s = sqrt(softplus(f)), softplus(f) = f above 20; rank by s + b; weights from s
                     (dsv41/xpu/csrc/dsv_moe_glue.sycl:163-193)
    A pick's weight is v * scaling / (sum of picked v + 1e-20) with renorm, v * scaling without.
    mul / res (sigmoid and sqrt_softplus, the dsv router's residency terms, dsv41/xpu/csrc/dsv_moe_glue.sycl:163-175):
    rank by s * mul + b + max(res, -1e30) instead, each float32 operation rounded on its own.
    Returns ids int32 [M, k] (descending rank, exact ties to the lower index) and w float32 [M, k]."""
    if score not in SCORES:
        raise ValueError(score)
    f = logits.astype(np.float32)
    b = None if bias is None else bias.astype(np.float32)[None, :]
    f64 = f.astype(np.float64)
    if score == "softmax":
        r = f if b is None else f + b
        g = r.astype(np.float64) if not bias_select_only else f64
        v = np.exp(g - g.max(-1, keepdims=True))
        v = v / v.sum(-1, keepdims=True)
    else:
        if score == "sigmoid":
            s32 = (np.float32(1) / (np.float32(1) + np.exp(-f))).astype(np.float32)
            v = 1.0 / (1.0 + np.exp(-f64))
        else:
            sp32 = np.where(f > 20, f, np.log1p(np.exp(np.minimum(f, 20)))).astype(np.float32)
            s32 = np.sqrt(sp32).astype(np.float32)
            v = np.sqrt(np.where(f64 > 20, f64, np.log1p(np.exp(np.minimum(f64, 20)))))
        r = (s32 + b) if b is not None else (f if score == "sigmoid" else s32)
        if mul is not None or res is not None:
            r = s32 * (np.float32(1) if mul is None else mul.astype(np.float32)[None, :])
            if b is not None:
                r = r + b
            if res is not None:
                r = r + np.maximum(res.astype(np.float32), np.float32(-1e30))[None, :]
    ids = topk_lowest_index(r, k)
    pv = np.take_along_axis(v, ids, -1)
    w = pv * scaling / (pv.sum(-1, keepdims=True) + 1e-20) if renorm else pv * scaling
    return ids.astype(np.int32), w.astype(np.float32)


def route_block(logits: np.ndarray, k: int, bias: np.ndarray | None = None, mul: np.ndarray | None = None,
                rows_per_block: int = 1, boost: float = 0.0, scaling: float = 1.0):
    """Verify-block routing (dsv41/xpu/csrc/dsv_moe_glue.sycl:194-240): sqrt-softplus s; rows of a block in order, an
    expert picked by an earlier row of the block ranks by s * mul * (1 + boost) + b, the others by s * mul + b (float32
    operations rounded one by one); weights from s (float64), renormalised (+1e-20) and scaled."""
    f = logits.astype(np.float32)
    M, E = f.shape
    sp32 = np.where(f > 20, f, np.log1p(np.exp(np.minimum(f, 20)))).astype(np.float32)
    s32 = np.sqrt(sp32).astype(np.float32)
    f64 = f.astype(np.float64)
    v = np.sqrt(np.where(f64 > 20, f64, np.log1p(np.exp(np.minimum(f64, 20)))))
    m32 = np.ones(E, np.float32) if mul is None else mul.astype(np.float32)
    up = np.float32(1) + np.float32(boost)
    ids = np.zeros((M, k), np.int32)
    w = np.zeros((M, k), np.float32)
    for b0 in range(0, M, rows_per_block):
        chosen = np.zeros(E, bool)
        for r in range(b0, b0 + rows_per_block):
            key = (s32[r] * m32).astype(np.float32) * np.where(chosen, up, np.float32(1)).astype(np.float32)
            if bias is not None:
                key = key + bias.astype(np.float32)
            order = topk_lowest_index(key.astype(np.float32)[None, :], k)[0]
            pv = v[r, order]
            ids[r] = order
            w[r] = pv * scaling / (pv.sum() + 1e-20)
            chosen[order] = True
    return ids, w


def router_logits(x: np.ndarray, W: np.ndarray, layout: str = "he", round_fp16: bool = False) -> np.ndarray:
    """logits[m, e] = sum_h x[m, h] W(h, e) in float64, returned as float32, or rounded to fp16 precision (the result of
    a matmul of two fp16 tensors, glm/xpu/glm_xpu/ops.py:183-184). layout "he": W [H, E] (gate_tensor); "eh": W [E, H]
    (a linear layer's weight, dsv41/xpu/csrc/dsv_moe_glue.sycl:442-470)."""
    Wm = W.astype(np.float64) if layout == "he" else W.astype(np.float64).T
    y = x.astype(np.float64) @ Wm
    return y.astype(np.float16).astype(np.float32) if round_fp16 else y.astype(np.float32)


def align(ids: np.ndarray, w: np.ndarray, E: int, pad: int = 1):
    """Pairs sorted by expert (stable: flat pair order within an expert), per active expert start / count / padded
    start, and the inverse map (exl3_moe.n128.sycl:691-734). Returns a dict of numpy arrays."""
    flat = ids.reshape(-1).astype(np.int64)
    topk = ids.shape[1]
    cnt = np.bincount(flat[flat >= 0], minlength=E)[:E]
    start = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    order = np.argsort(np.where(flat >= 0, flat, E), kind="stable")[: int(cnt.sum())]
    act = np.nonzero(cnt)[0]
    pc = (cnt + pad - 1) // pad * pad
    pstart = np.concatenate([[0], np.cumsum(pc)[:-1]])
    pair_of = np.full(flat.size, -1, dtype=np.int64)
    pair_of[order] = np.arange(order.size)
    return dict(act_expert=act.astype(np.int32), act_start=start[act].astype(np.int32),
                act_cnt=cnt[act].astype(np.int32), n_act=np.int32(act.size), act_pstart=pstart[act].astype(np.int32),
                pair_tok=(order // topk).astype(np.int32), pair_w=w.reshape(-1)[order].astype(np.float32),
                pair_of=pair_of.astype(np.int32), count=cnt.astype(np.int32))


# ------------------------------------------------------------------------------------------------ expert blob


def planar4_words(tr: np.ndarray, K: int) -> np.ndarray:
    """int16 trellis [rows, tiles, 16K] -> uint32 words in the reference's PLANAR4 order: a tile is G periods of D
    words (D = K / gcd(K, 32), G = 8K / D); groups of 4 consecutive tiles are stored plane by plane, [D][4][G]
    (moe_offload.py:68-78, pack_store.py:41-54). D = 1 (K = 2, 4, 8) leaves the words in tile order."""
    rows, tiles, _ = tr.shape
    D = K // math.gcd(K, 32)
    G = 8 * K // D
    w = np.ascontiguousarray(tr).view(np.uint32).reshape(rows, tiles // 4, 4, G, D)
    return w.transpose(0, 1, 4, 2, 3).reshape(-1)


def reference_blob(gate: dict, up: dict, down: dict, K: int) -> np.ndarray:
    """The reference's expert blob bytes (pack_expert, moe_offload.py:81-94): planar4(gate|up trellis concatenated
    along the columns), planar4(down), then gate.suh, up.suh, gate.svh, up.svh, down.suh, down.svh (fp16)."""
    gu = np.concatenate([gate["trellis"], up["trellis"]], axis=1)
    parts = [planar4_words(gu, K).view(np.uint8), planar4_words(down["trellis"], K).view(np.uint8)]
    for v in (gate["suh"], up["suh"], gate["svh"], up["svh"], down["suh"], down["svh"]):
        parts.append(np.ascontiguousarray(v, dtype=np.float16).view(np.uint8))
    return np.concatenate(parts)


def reference_geom_bytes(H: int, I: int, K: int) -> int:
    """Geom::blob() (exl3_moe.n128.sycl:56-68): gate|up and down trellis words, then six fp16 vectors."""
    W = 8 * K
    return (H // 16) * (2 * I // 16) * W * 4 + (I // 16) * (H // 16) * W * 4 + 2 * (3 * H + 3 * I)
