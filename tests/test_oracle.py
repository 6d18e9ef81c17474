"""Pins the CPU oracle (oracle/exl3_oracle.py) before it is trusted as the checker.

The reference holds no golden vectors for this path (its parity tests need checkpoints and the un-vendored exllamav3
testlib), so every oracle function is pinned by an independent statement or by mathematics:
  * codebook: six textual statements of mul1 in the reference must agree over all 65536 states, plus the value
    invariants the reference states (913 distinct values, range [-3.453, 3.348]);
  * tile permutation: three statements (bit-field, ring, inverse) agree and form a bijection;
  * window extraction + whole-tile decode: a brute-force C decoder that materialises the ring bit by bit;
  * Hadamard: orthogonality, basis vectors, involution, dense +-1 matmul;
  * linear: the transform path equals x @ W with W = diag(suh) Hblk W_hat Hblk diag(svh) built the other way round;
  * routing / align: closed-form invariants and hand-built ties;
  * MoE: linearity in the routing weights, the dense-weight form of every expert, slot bookkeeping.
"""
import ctypes
import math
import os

import numpy as np
import pytest

from oracle import exl3_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BF_LIB = os.path.join(ROOT, "oracle", "_build", "libexl3_oracle.so")


@pytest.fixture(scope="module")
def bf():
    if not os.path.exists(BF_LIB):
        import subprocess
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
    L = ctypes.CDLL(BF_LIB)
    L.exl3_bf_mul1.restype = ctypes.c_uint16
    L.exl3_bf_mul1.argtypes = [ctypes.c_uint32]
    L.exl3_bf_f64_to_f16.restype = ctypes.c_uint16
    L.exl3_bf_f64_to_f16.argtypes = [ctypes.c_double]
    L.exl3_bf_reconstruct.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    return L


def bf_reconstruct(bf, tr):
    tk, tn, w = tr.shape
    out = np.empty((tk * 16, tn * 16), dtype=np.uint16)
    tr = np.ascontiguousarray(tr)
    assert bf.exl3_bf_reconstruct(tr.ctypes.data, tk, tn, w // 16, out.ctypes.data) == 0
    return out


# ------------------------------------------------------------------------------------------------ codebook

def test_lut_invariants():
    lut = O.mul1_lut()
    v = lut.astype(np.float64)
    assert np.unique(lut.view(np.uint16)).size == 913
    assert v.min() == -3.453125 and v.max() == 3.34765625
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    # the two fp16 constants are the bit patterns the reference names (0x1EEE, 0xC931)
    assert np.array([O.K_INV], np.float16).view(np.uint16)[0] == 0x1EEE
    assert np.array([O.K_BIAS], np.float16).view(np.uint16)[0] == 0xC931


def test_lut_statements_agree(bf):
    st = np.arange(65536, dtype=np.uint64)
    lut = O.mul1_lut().view(np.uint16)
    x = (st * 0x83DCD12D) & 0xFFFFFFFF
    # (1) MUL16 split of the multiply, glm/xpu/csrc/exl3_esimd.h:47-53
    x16 = (st * 0xD12D + (((st * 0x83DC) & 0xFFFF) << 16)) & 0xFFFFFFFF
    assert np.array_equal(x, x16)
    # (2) dp4a form: 0x6400 + byte sum is the fp16 bit pattern of 1024 + byte sum (exl3_esimd.h:57-59)
    s = sum(((x >> (8 * i)) & 0xFF) for i in range(4))
    h_bits = (0x6400 + s).astype(np.uint16)
    assert np.array_equal(h_bits.view(np.float16).astype(np.float64), 1024.0 + s)
    # (3) fp16 fma with one rounding == fp32 affine (exact) rounded once (triton_kernels.py:38-42, exl3_tri.py:38-43)
    h = h_bits.view(np.float16).astype(np.float32)
    v32 = (h * np.float32(O.K_INV) + np.float32(O.K_BIAS))
    exact = h.astype(np.float64) * O.K_INV + O.K_BIAS
    assert np.array_equal(v32.astype(np.float64), exact)            # the fp32 affine is exact
    assert np.array_equal(v32.astype(np.float16).view(np.uint16), lut)
    # (4) glm/xpu/tests/units.py:45-49 form: ((1024 + s).double() * K_INV - 10.3828125).float().half()
    v4 = ((1024 + s).astype(np.float64) * 0.00676727294921875 - 10.3828125).astype(np.float32).astype(np.float16)
    assert np.array_equal(v4.view(np.uint16), lut)
    # (5) brute-force C: byte loop + hand-written round-to-nearest-even
    sample = np.random.default_rng(1).integers(0, 65536, 4096)
    assert all(bf.exl3_bf_mul1(int(t)) == lut[t] for t in sample)
    assert all(bf.exl3_bf_mul1(int(t)) == lut[t] for t in range(0, 65536, 97))


def test_bruteforce_f16_rounding_matches_numpy(bf):
    # the C converter used by the brute-force decoder is itself checked against numpy on hard cases
    vals = np.concatenate([np.random.default_rng(2).normal(0, 4, 2000), [0.0, -0.0, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                           65504.0, 65519.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, -2.5e-5, 6.1e-5]])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([bf.exl3_bf_f64_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(ref, got)


# ------------------------------------------------------------------------------------------------ layout

def test_permutation_statements_agree():
    row, col = O.pos_row_col()
    t = np.arange(256)
    # ring form (dsv41/xpu/dsv_xpu/exl3_tri.py:4-9)
    tt, j = t // 8, t % 8
    r2 = (tt % 4) * 2 + (j & 1) + 8 * ((j >> 1) & 1)
    c2 = tt // 4 + 8 * ((j >> 2) & 1)
    assert np.array_equal(row, r2) and np.array_equal(col, c2)
    # inverse form (glm/xpu/exl3xpu/triton_kernels.py:4-7): t = 32(c&7) + 8((r>>1)&3) + 4(c>>3) + 2(r>>3) + (r&1)
    inv = 32 * (col & 7) + 8 * ((row >> 1) & 3) + 4 * (col >> 3) + 2 * (row >> 3) + (row & 1)
    assert np.array_equal(inv, t)
    # bijection onto the 16 x 16 tile
    assert np.unique(row * 16 + col).size == 256


@pytest.mark.parametrize("K", range(1, 9))
def test_decode_vs_bruteforce(bf, K):
    rng = np.random.default_rng(100 + K)
    tr = rng.integers(-32768, 32768, size=(3, 4, 16 * K), dtype=np.int16)
    assert np.array_equal(O.reconstruct(tr, K).view(np.uint16), bf_reconstruct(bf, tr))


@pytest.mark.parametrize("K", range(1, 9))
def test_fast_decoder_matches_numpy_and_bruteforce(bf, K):
    """The C decoder used for full-size parity cases (oracle/trellis_fast.c) is bit-identical to the NumPy statement
    and the bit-by-bit decoder, whole matrices and column slices."""
    rng = np.random.default_rng(200 + K)
    tr = rng.integers(-32768, 32768, size=(5, 24, 16 * K), dtype=np.int16)
    ref = O.reconstruct(tr, K)
    assert np.array_equal(O.reconstruct_fast(tr, K).view(np.uint16), ref.view(np.uint16))
    assert np.array_equal(ref.view(np.uint16), bf_reconstruct(bf, tr))
    assert np.array_equal(O.reconstruct_fast(tr, K, 128, 128).view(np.uint16), ref[:, 128:256].view(np.uint16))


def test_fast_mixed_decoder_matches_numpy():
    rng = np.random.default_rng(5)
    k, n = 96, 160
    tk, tn = k // 16, n // 16
    kmap = rng.integers(1, 9, tk * tn).astype(np.uint8)
    woff = np.concatenate([[0], np.cumsum(kmap.astype(np.int64) * 8)])
    words = rng.integers(0, 2 ** 32, int(woff[-1]), dtype=np.uint64).astype(np.uint32)
    a = O.reconstruct_mixed(words, kmap, woff, k, n)
    b = O.reconstruct_mixed_fast(words, kmap, woff, k, n)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("K", [1, 2, 3, 4, 8])
def test_fast_matmul_matches_dense_product(K):
    """x @ W_hat through the C decoder (used by Proj for large matrices) equals the float64 product with the NumPy
    reconstruction, uniform and per-tile K, for 1 and 19 rows (the C loop takes rows 16 at a time)."""
    rng = np.random.default_rng(300 + K)
    k, n = 128, 96
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
    kmap = rng.integers(1, 9, (k // 16) * (n // 16)).astype(np.uint8)
    woff = np.concatenate([[0], np.cumsum(kmap.astype(np.int64) * 8)])
    words = rng.integers(0, 2 ** 32, int(woff[-1]), dtype=np.uint64).astype(np.uint32)
    for m in (1, 19):
        x = rng.normal(0, 1, (m, k))
        ref = x @ O.reconstruct(tr, K).astype(np.float64)
        np.testing.assert_allclose(O.matmul_fast(x, trellis=tr, K=K), ref, rtol=1e-12, atol=1e-12)
        refm = x @ O.reconstruct_mixed(words, kmap, woff, k, n).astype(np.float64)
        np.testing.assert_allclose(O.matmul_fast(x, words=words, kmap=kmap, woff=woff), refm, rtol=1e-12, atol=1e-12)


def test_window_special_cases(bf):
    # K = 8: windows are byte aligned; K = 1: 15 of 16 bits of early windows come from the ring's end
    for K in (1, 8, 16 // 2, 3):
        tr = np.zeros((1, 1, 16 * K), dtype=np.int16)
        tr.view(np.uint32)[0, 0, -1] = 0x0000FFFF          # ones at the very end of the ring
        W = O.reconstruct(tr, K)
        assert np.array_equal(W.view(np.uint16), bf_reconstruct(bf, tr))
        st = O.tile_states(tr.view(np.uint32)[0, 0], K)
        # position 0's window starts in the last word: it sees (16 - K) trailing ones then K zeros
        assert st[0] == ((0xFFFF << K) & 0xFFFF)


def test_reconstruct_slice_consistency():
    rng = np.random.default_rng(3)
    tr = rng.integers(-32768, 32768, size=(4, 24, 48), dtype=np.int16)
    W = O.reconstruct(tr, 3)
    assert np.array_equal(O.reconstruct(tr, 3, 128, 256), W[:, 128:384])


def test_mixed_k_reconstruct_matches_uniform():
    rng = np.random.default_rng(4)
    k, n = 64, 96
    tk, tn = k // 16, n // 16
    kmap = rng.integers(1, 3, tk * tn).astype(np.uint8)
    woff = np.concatenate([[0], np.cumsum(kmap.astype(np.int64) * 8)])
    words = rng.integers(0, 2 ** 32, int(woff[-1]), dtype=np.uint64).astype(np.uint32)
    W = O.reconstruct_mixed(words, kmap, woff, k, n)
    for i in range(tk * tn):
        a, b = divmod(i, tn)
        K = int(kmap[i])
        tile = words[woff[i]:woff[i] + 8 * K].view(np.int16).reshape(1, 1, 16 * K)
        assert np.array_equal(W[16 * a:16 * a + 16, 16 * b:16 * b + 16], O.reconstruct(tile, K))


# ------------------------------------------------------------------------------------------------ Hadamard

def test_hadamard_properties():
    H = O.sylvester128()
    assert np.array_equal(H @ H.T, 128 * np.eye(128))
    i = np.arange(128)
    pc = np.array([bin(v).count("1") for v in range(128)])
    assert np.array_equal(H, (-1.0) ** pc[np.bitwise_and.outer(i, i)])
    e = np.eye(128)[37:38]
    assert np.array_equal(O.had_blocks(e)[0], H[37])
    x = np.random.default_rng(5).normal(size=(3, 256))
    y = O.had_r_128(O.had_r_128(x.astype(np.float32)), None)   # involution up to fp32 rounding
    assert np.allclose(y, x, atol=1e-5)


def test_had_r_128_rounding_points():
    rng = np.random.default_rng(6)
    x = rng.normal(size=(4, 256)).astype(np.float16)
    pre = (rng.integers(0, 2, 256) * 2 - 1).astype(np.float16) * np.float16(0.37)
    y = O.had_r_128(x, pre=pre)
    xp = (x.astype(np.float32) * pre.astype(np.float32)).astype(np.float16)     # x * pre rounded first
    ref = ((xp.astype(np.float64).reshape(-1, 128) @ O.sylvester128()) / math.sqrt(128)).reshape(x.shape)
    assert np.array_equal(y, ref.astype(np.float16))
    post = pre
    y2 = O.had_r_128(x, post=post)
    ref2 = (((x.astype(np.float64).reshape(-1, 128) @ O.sylvester128()) / math.sqrt(128)).reshape(x.shape)
            .astype(np.float16).astype(np.float32) * post.astype(np.float32)).astype(np.float16)
    assert np.array_equal(y2, ref2)
    # both given: only pre applies
    assert np.array_equal(O.had_r_128(x, pre=pre, post=post), y)


# ------------------------------------------------------------------------------------------------ linear

def _lin(k, n, K, seed):
    rng = np.random.default_rng(seed)
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
    suh = ((rng.integers(0, 2, k) * 2 - 1) * 0.75).astype(np.float16)
    svh = ((rng.integers(0, 2, n) * 2 - 1) / math.sqrt(k)).astype(np.float16)
    return tr, suh, svh


@pytest.mark.parametrize("K", [2, 4])
def test_linear_equals_dense_weight(K):
    tr, suh, svh = _lin(256, 384, K, 7)
    x = np.random.default_rng(8).normal(size=(3, 256)).astype(np.float16)
    Wd = O.dense_weight(tr, suh, svh, K)
    ref = x.astype(np.float64) @ Wd
    # transform path without the fp16 rounding points == dense form, to fp64 precision
    xh = O.had_blocks(x.astype(np.float64) * suh.astype(np.float64)) / math.sqrt(128)
    y = O.had_blocks(xh @ O.reconstruct(tr, K).astype(np.float64)) / math.sqrt(128) * svh.astype(np.float64)
    assert np.abs(y - ref).max() < 1e-9 * np.abs(ref).max()
    # with the reference rounding points: within the fp16 rounding of the activations
    y32 = O.exl3_linear(x, tr, suh, svh, K, np.float32)
    assert np.abs(y32 - ref).max() / np.abs(ref).max() < 2e-3


def test_linear_tiny_bruteforce(bf):
    tr, suh, svh = _lin(128, 128, 3, 9)
    W_bf = bf_reconstruct(bf, tr).view(np.float16).astype(np.float64)
    Hb = O.sylvester128() / math.sqrt(128)
    Wd = suh.astype(np.float64)[:, None] * (Hb @ W_bf @ Hb) * svh.astype(np.float64)[None, :]
    x = np.random.default_rng(10).normal(size=(2, 128)).astype(np.float16)
    y = O.exl3_linear(x, tr, suh, svh, 3, np.float32)
    ref = x.astype(np.float64) @ Wd
    assert np.abs(y - ref).max() / np.abs(ref).max() < 2e-3


def test_mgemm_slots_filter_and_weighted_sum():
    """exl3_mgemm restatement pinned by independent forms: each slot equals x @ dense_weight of its matrix (closed
    form), the [min, max) filter equals a manual remap of the indices, and the weighted token sum equals the weighted
    sum of the dense products."""
    mats = [_lin(128, 256, 2, 30 + q) for q in range(4)]
    dense = [O.dense_weight(tr, suh, svh, 2) for tr, suh, svh in mats]
    rng = np.random.default_rng(31)
    A = rng.normal(size=(6, 2, 128)).astype(np.float16)           # a_batches = slots = 6
    idx = np.array([2, -1, 0, 3, 7, 1])                           # 7 is out of range: skipped like -1
    C0 = np.full((6, 2, 256), 5.0, np.float32)
    y = O.mgemm(A, mats, 2, idx, C=C0)
    for j, q in enumerate(idx):
        if 0 <= q < 4:
            ref = A[j].astype(np.float64) @ dense[q]
            assert np.abs(y[j] - ref).max() / np.abs(ref).max() < 2e-3, j
        else:
            assert (y[j] == 5.0).all(), j
    # filter [1, 3): indices 2 -> 1, 1 -> 0, others skipped
    yf = O.mgemm(A, mats, 2, idx, min_index=1, max_index=3, C=C0)
    remap = np.array([1, -1, -1, -1, -1, 0])
    assert np.array_equal(yf, O.mgemm(A, mats, 2, remap, C=C0))
    # weighted, 2 tokens x 3 slots, A per token
    At = A[:2]
    w = np.array([0.5, 1.25, -2.0, 0.75, 3.0, -0.5], np.float16)
    yw = O.mgemm(At, mats, 2, idx, w, num_tokens=2, out_dtype=np.float64)
    for t in range(2):
        ref = sum(float(w[j]) * (At[t].astype(np.float64) @ dense[idx[j]])
                  for j in range(3 * t, 3 * t + 3) if 0 <= idx[j] < 4)
        assert np.abs(yw[t] - ref).max() / np.abs(ref).max() < 2e-3, t


# ------------------------------------------------------------------------------------------------ routing / align

def test_route_softmax_topk():
    rng = np.random.default_rng(11)
    logits = rng.normal(size=(5, 64)).astype(np.float32)
    logits[0, [3, 9, 20]] = 4.0                         # exact ties: lower index first
    ids, w = O.route_softmax_topk(logits, 4)
    assert list(ids[0, :3]) == [3, 9, 20]
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    for r in range(5):
        top = np.argsort(-logits[r], kind="stable")[:4]
        assert list(ids[r]) == list(top)
        assert np.allclose(w[r], p[r, top] / p[r, top].sum(), rtol=1e-6)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)
    bias = np.zeros(64, np.float32)
    bias[50] = 100.0
    ids_b, w_b = O.route_softmax_topk(logits, 4, bias)
    assert (ids_b[:, 0] == 50).all() and (w_b[:, 0] > 0.99).all()


@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrt_softplus"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_route_topk_scorings_against_torch(score, with_bias):
    """Each scoring against an independent torch statement of the reference formula (torch.sigmoid / softplus /
    softmax and torch.topk): trellis-serve.patch:403-424 (softmax, `cold` as a selection-only bias),
    glm/xpu/glm_xpu/ops.py:186-191 (sigmoid), dsv41/xpu/csrc/dsv_moe_glue.sycl:163-193 (sqrt-softplus)."""
    import torch
    g = torch.Generator().manual_seed(11 + 3 * with_bias + len(score))
    logits = torch.randn(9, 96, generator=g) * 3
    bias = torch.randn(96, generator=g) * 0.5 if with_bias else None
    k, scaling = 6, 2.5
    f = logits.double()
    if score == "softmax":
        v = torch.softmax(f, -1)
        key = f + bias.double() if with_bias else f
    elif score == "sigmoid":
        v = torch.sigmoid(f)
        key = v + bias.double() if with_bias else f
    else:
        v = torch.sqrt(torch.nn.functional.softplus(f, threshold=20))
        key = v + bias.double() if with_bias else v
    idx = torch.topk(key, k, dim=-1, sorted=True).indices
    pv = v.gather(-1, idx)
    w_ref = pv * scaling / (pv.sum(-1, keepdim=True) + 1e-20)
    ids, w = O.route_topk(logits.numpy(), k, None if bias is None else bias.numpy(), score, True, scaling,
                          bias_select_only=True)
    assert np.array_equal(ids, idx.numpy())
    assert np.abs(w - w_ref.numpy()).max() <= 1e-6 * scaling
    # without renormalisation the weights are the scores themselves (times scaling)
    _, w_raw = O.route_topk(logits.numpy(), k, None if bias is None else bias.numpy(), score, False, scaling,
                            bias_select_only=True)
    assert np.abs(w_raw - (pv * scaling).numpy()).max() <= 1e-6 * float(pv.max()) * scaling


@pytest.mark.parametrize("score", ["sigmoid", "sqrt_softplus"])
def test_route_topk_residency_terms(score):
    """mul / res ranking (the dsv router's residency terms) pinned by properties: without them it is the plain router;
    a uniform positive mul without bias keeps the plain order; -inf residency never picks an expert while k others
    remain, and equals dropping those experts from the plain ranking; weights always come from the unmodified score."""
    rng = np.random.default_rng(41)
    lg = rng.normal(size=(6, 40)).astype(np.float32) * 2
    b = (rng.normal(size=40) * 0.3).astype(np.float32)
    ids0, w0 = O.route_topk(lg, 6, b, score)
    ids1, w1 = O.route_topk(lg, 6, b, score, mul=None, res=np.zeros(40, np.float32))
    assert np.array_equal(ids0, ids1) and np.array_equal(w0, w1)
    ids2, _ = O.route_topk(lg, 6, None, score, mul=np.full(40, 2.0, np.float32))
    ids3, _ = O.route_topk(lg, 6, None, "sqrt_softplus" if score == "sqrt_softplus" else score)
    if score == "sqrt_softplus":
        assert np.array_equal(ids2, ids3)
    res = np.where(np.arange(40) % 3 == 0, -np.inf, 0.0).astype(np.float32)
    ids4, w4 = O.route_topk(lg, 6, b, score, res=res)
    assert not np.isin(ids4, np.arange(0, 40, 3)).any()
    keep = np.arange(40)[np.arange(40) % 3 != 0]
    idk, wk = O.route_topk(lg[:, keep], 6, b[keep], score)
    assert np.array_equal(ids4, keep[idk]) and np.allclose(w4, wk, rtol=1e-6)


def _logits_for_sqrt_softplus(s):
    """Logits f with sqrt(softplus(f)) = s (f = log(expm1(s^2)))."""
    return np.log(np.expm1(np.asarray(s, np.float64) ** 2)).astype(np.float32)


def test_route_residency_terms_hand_computed():
    """The residency form ranks by s * mul + b (+ res), hand-computed on three experts: s = (0.5, 0.75, 0.1),
    mul = (3, 1, 1), b = (-0.2, 0.2, 0) give keys (1.3, 0.95, 0.1), so the picks are (0, 1) with weights
    s / (0.5 + 0.75) = (0.4, 0.6). (s + b) * mul would give (0.9, 0.95, 0.1) and pick (1, 0); s * (mul + b) gives
    (1.4, 0.95, 0.1) and agrees, so a second case separates it: res = (-0.4, 0, 0) makes the keys (0.9, 0.95, 0.1),
    picks (1, 0) with weights (0.6, 0.4), where s * (mul + b) + res = (1.0, 0.95, 0.1) would keep (0, 1)."""
    lg = _logits_for_sqrt_softplus([0.5, 0.75, 0.1])[None, :]
    mul = np.array([3, 1, 1], np.float32)
    b = np.array([-0.2, 0.2, 0.0], np.float32)
    ids, w = O.route_topk(lg, 2, b, "sqrt_softplus", mul=mul)
    assert ids.tolist() == [[0, 1]]
    assert np.allclose(w, [[0.4, 0.6]], atol=1e-6)
    ids, w = O.route_topk(lg, 2, b, "sqrt_softplus", mul=mul, res=np.array([-0.4, 0, 0], np.float32))
    assert ids.tolist() == [[1, 0]]
    assert np.allclose(w, [[0.6, 0.4]], atol=1e-6)


def test_route_block_boost_hand_computed():
    """Verify-block boost is multiplicative, s * mul * (1 + bb) + b, hand-computed on two experts in one block of two
    rows: row 0 (s = 1.5, 0.3) picks expert 0; row 1 has s = (0.5, 1.2). With mul = 1 and bb = 1 expert 0's key is
    0.5 * 2 = 1.0 < 1.2, so row 1 picks expert 1 (an additive boost s + bb = 1.5 would pick expert 0); with bb = 2 it
    is 1.5 > 1.2 and row 1 picks expert 0. With mul = (2, 1) and bb = 0.25 it is 0.5 * 2 * 1.25 = 1.25 > 1.2: expert 0
    (s * (mul + bb) = 1.125 would pick expert 1). The weights are the plain s renormalised over one pick: 1."""
    lg = np.stack([_logits_for_sqrt_softplus([1.5, 0.3]), _logits_for_sqrt_softplus([0.5, 1.2])])
    zero = np.zeros(2, np.float32)
    for mul, bb, want in ((None, 1.0, 1), (None, 2.0, 0), (np.array([2, 1], np.float32), 0.25, 0),
                          (np.array([2, 1], np.float32), 0.1, 1)):
        ids, w = O.route_block(lg, 1, zero, mul, 2, bb)
        assert ids[:, 0].tolist() == [0, want], (mul, bb)
        assert np.allclose(w, 1.0)
    # a bias adds after the boost: b = (0, 0.35) lifts expert 1 to 1.55 over 1.5 at bb = 2
    ids, _ = O.route_block(lg, 1, np.array([0, 0.35], np.float32), None, 2, 2.0)
    assert ids[:, 0].tolist() == [0, 1]


def test_route_block_properties():
    """Verify-block routing pinned by properties: no boost (or blocks of one row) is the plain sqrt-softplus router row
    by row; a boost large enough makes every later row of a block take the first row's experts; the weights always
    come from the plain score of the picks."""
    rng = np.random.default_rng(43)
    lg = rng.normal(size=(8, 64)).astype(np.float32) * 2
    b = (rng.normal(size=64) * 0.2).astype(np.float32)
    mul = (1 + rng.random(64)).astype(np.float32)
    pi, pw = O.route_topk(lg, 5, b, "sqrt_softplus", mul=mul)
    for S, boost in ((4, 0.0), (1, 3.0)):
        bi, bw = O.route_block(lg, 5, b, mul, S, boost)
        assert np.array_equal(bi, pi) and np.allclose(bw, pw, rtol=1e-6)
    bi, bw = O.route_block(lg, 5, b, None, 4, 1e4)
    for blk in range(2):
        first = set(bi[4 * blk].tolist())
        assert all(set(bi[4 * blk + r].tolist()) == first for r in range(4))
    pi0, pw0 = O.route_topk(lg, 5, None, "sqrt_softplus")
    v = np.sqrt(np.log1p(np.exp(lg.astype(np.float64))))
    for r in range(8):
        pv = v[r, bi[r]]
        assert np.allclose(bw[r], pv / (pv.sum() + 1e-20), rtol=1e-6)


def test_route_topk_softmax_bias_both_is_route_softmax_topk():
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((7, 200)).astype(np.float32)
    bias = rng.standard_normal(200).astype(np.float32)
    a = O.route_softmax_topk(logits, 8, bias)
    b = O.route_topk(logits, 8, bias, "softmax")
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # selection-only bias: same picks, weights from the unbiased softmax
    c = O.route_topk(logits, 8, bias, "softmax", bias_select_only=True)
    assert np.array_equal(a[0], c[0])
    p = np.exp(logits.astype(np.float64))
    p /= p.sum(-1, keepdims=True)
    pv = np.take_along_axis(p, c[0].astype(np.int64), -1)
    assert np.allclose(c[1], pv / pv.sum(-1, keepdims=True), rtol=1e-6)


def test_router_logits_layouts_and_fp16_rounding():
    import torch
    g = torch.Generator().manual_seed(21)
    x = torch.randn(5, 256, generator=g).half()
    W = (torch.randn(256, 40, generator=g) * 0.1).half()
    ref = (x.double() @ W.double()).numpy()
    he = O.router_logits(x.numpy(), W.numpy(), "he")
    eh = O.router_logits(x.numpy(), W.T.contiguous().numpy(), "eh")
    assert np.array_equal(he, eh) and np.abs(he - ref).max() <= 1e-6 * np.abs(ref).max()
    r16 = O.router_logits(x.numpy(), W.numpy(), "he", round_fp16=True)
    assert np.array_equal(r16, ref.astype(np.float16).astype(np.float32))
    # torch's own fp16 matmul (fp32 accumulation, one rounding) agrees within one fp16 ulp
    t16 = torch.matmul(x, W).float().numpy()
    d = np.abs(t16.astype(np.float16).view(np.int16).astype(np.int32) - r16.astype(np.float16).view(np.int16))
    assert d.max() <= 1


def test_align_invariants():
    rng = np.random.default_rng(12)
    ids = rng.integers(0, 16, size=(9, 4)).astype(np.int32)
    w = rng.random((9, 4)).astype(np.float32)
    a = O.align(ids, w, 16, pad=4)
    cnt = np.bincount(ids.reshape(-1), minlength=16)
    assert np.array_equal(a["count"], cnt)
    assert np.array_equal(a["act_expert"], np.nonzero(cnt)[0])
    assert np.array_equal(a["act_start"], np.concatenate([[0], np.cumsum(cnt)])[a["act_expert"]])
    assert (a["act_pstart"] % 4 == 0).all()
    flat = ids.reshape(-1)
    for i in range(flat.size):
        pos = a["pair_of"][i]
        assert a["pair_tok"][pos] == i // 4 and a["pair_w"][pos] == w.reshape(-1)[i]
    assert np.unique(a["pair_of"]).size == flat.size


# ------------------------------------------------------------------------------------------------ MoE

def _experts(E, H, I, K, seed):
    out = []
    for e in range(E):
        ps = []
        for j, (k, n) in enumerate(((H, I), (H, I), (I, H))):
            tr, suh, svh = _lin(k, n, K, seed + 10 * e + j)
            ps.append(O.Proj(suh, svh, trellis=tr, K=K))
        out.append(tuple(ps))
    return out


def test_moe_layer_structure():
    H, I, E = 256, 128, 5
    ex = _experts(E, H, I, 2, 300)
    rng = np.random.default_rng(13)
    x = rng.normal(size=(3, H)).astype(np.float16)
    ids = np.array([[0, 3], [3, 3], [4, 1]], np.int32)      # duplicate expert within a token
    w = rng.random((3, 2)).astype(np.float32)
    out = O.moe_layer(x, ex, ids, w, O.ACT_SILU)
    out2 = O.moe_layer(x, ex, ids, 2 * w, O.ACT_SILU)
    assert np.allclose(out2, 2 * out, rtol=1e-6, atol=1e-6)  # linear in the routing weights
    # each expert against its dense-weight form (fp64, no fp16 rounding points)
    dense = []
    for g, u, d in ex:
        dense.append([O.dense_weight(p.trellis, p.suh, p.svh, p.K) for p in (g, u, d)])
    ref = np.zeros((3, H))
    for t in range(3):
        for j in range(2):
            Wg, Wu, Wd = dense[ids[t, j]]
            xg = x[t].astype(np.float64)
            a = O.act_mul(xg @ Wg, xg @ Wu, O.ACT_SILU)
            ref[t] += w[t, j] * (a @ Wd)
    assert np.abs(out - ref).max() / np.abs(ref).max() < 5e-3
    # inactive slots contribute nothing
    ids_m = ids.copy()
    ids_m[2, 1] = -1
    w_m = w.copy()
    w_m[2, 1] = 0
    assert np.allclose(O.moe_layer(x, ex, ids_m, w, O.ACT_SILU), O.moe_layer(x, ex, ids, w_m, O.ACT_SILU), atol=1e-6)


def _act_points():
    """A dense grid over [-20, 20], the fp16 extremes (largest finite, smallest normal and subnormal) of both signs,
    and N(0, 3) samples: float64."""
    fp16 = np.array([65504.0, 6.103515625e-05, 5.960464477539063e-08, 1e-3, 0.5, 8.0, 11.0])
    rng = np.random.default_rng(7)
    return np.concatenate([np.linspace(-20.0, 20.0, 40001), fp16, -fp16, [0.0], rng.normal(0, 3, 5000)])


def test_act_mul_matches_torch_gelu_tanh_and_silu():
    """GELU-tanh and SiLU (with and without the act_limit clamp) against torch.nn.functional in float64 (the SiLU
    clamp form of ext-op-inventory.md:944-956: min(silu(g), L) * clamp(u, -L, L)). torch is an independent
    statement of both functions (gelu(approximate='tanh'), silu)."""
    import torch
    import torch.nn.functional as F
    g = _act_points()
    u = np.random.default_rng(8).normal(0, 2, g.size)
    tg, tu = torch.from_numpy(g), torch.from_numpy(u)
    ref_gelu = (F.gelu(tg, approximate="tanh") * tu).numpy()
    ref_silu = (F.silu(tg) * tu).numpy()
    for L in (1.0, 10.0):
        ref_clamp = (torch.clamp(F.silu(tg), max=L) * torch.clamp(tu, -L, L)).numpy()
        np.testing.assert_allclose(O.act_mul(g, u, O.ACT_SILU, L), ref_clamp, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(O.act_mul(g, u, O.ACT_GELU_TANH), ref_gelu, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(O.act_mul(g, u, O.ACT_SILU), ref_silu, rtol=1e-12, atol=1e-14)
    # the check separates the plausible mistakes: exact-erf GELU, the cubic coefficient off by 10x, SiLU with the
    # clamp applied before the activation (sglang's swiglu_clamped), all differ by far more than the tolerance
    erf = (F.gelu(tg) * tu).numpy()
    c = math.sqrt(2.0 / math.pi)
    bad_coef = 0.5 * g * (1.0 + np.tanh(c * (g + 0.44715 * g ** 3))) * u
    pre_clamp = (F.silu(torch.clamp(tg, max=1.0)) * torch.clamp(tu, -1.0, 1.0)).numpy()
    for wrong, good in ((erf, ref_gelu), (bad_coef, ref_gelu), (pre_clamp, O.act_mul(g, u, O.ACT_SILU, 1.0))):
        assert np.abs(wrong - good).max() > 1e-5
