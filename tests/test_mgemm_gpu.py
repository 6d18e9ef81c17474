"""GPU parity of exl3_mgemm (multi-matrix EXL3 linear over int64 address tables) against the oracle's restatement.

Bars: every slot within max|y - r| / max|r| <= 2e-3 of the float64-accumulated oracle (as the dense linear); skipped
slots leave C bit-identical; a single slot is bit-identical to exl3_gemm (same kernel, same split); an MoE layer
composed from mgemm calls (gate, up, act, weighted down) within 2e-3 of the oracle's MoE layer.
"""
import numpy as np
import pytest
import torch

from moe_util import max_rel

pytestmark = pytest.mark.gpu
MAX_REL = 2e-3


def _mats(exl3, synth, nmat, k, n, K, seed):
    cpu = [synth.linear(k, n, K, seed + q) for q in range(nmat)]
    lins = [exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), K, None, False, True, None) for tr, suh, svh in cpu]
    ora = [(tr.numpy(), suh.numpy(), svh.numpy()) for tr, suh, svh in cpu]
    return lins, ora


@pytest.fixture(scope="module")
def synth():
    import importlib
    return importlib.import_module("b70-inference_amd.synth")


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("m", [1, 3, 12])
@pytest.mark.parametrize("cdt", [torch.float16, torch.float32])
def test_mgemm_slots_broadcast(exl3, oracle, synth, K, m, cdt):
    """No indices: slot j runs matrix j on the broadcast A (the fused gate|up form)."""
    lins, ora = _mats(exl3, synth, 3, 256, 384, K, 500 + K)
    B, S, V = exl3.mgemm_tables(lins)
    A = torch.randn(1, m, 256, generator=torch.Generator().manual_seed(m)).half()
    C = torch.empty(3, m, 384, dtype=cdt, device="cuda")
    exl3.exl3_mgemm(A.cuda(), B, C, S, None, V, None, None, K)
    ref = oracle.mgemm(A.numpy(), ora, K)
    for j in range(3):
        assert max_rel(C[j].float().cpu().numpy(), ref[j]) <= MAX_REL, j


@pytest.mark.parametrize("m", [1, 9])
def test_mgemm_indices_skip_and_filter(exl3, oracle, synth, m):
    """Negative, out-of-range and filtered-out indices leave their C rows untouched; kept ones are rebased."""
    lins, ora = _mats(exl3, synth, 5, 256, 256, 3, 600)
    B, S, V = exl3.mgemm_tables(lins)
    g = torch.Generator().manual_seed(7)
    A = torch.randn(6, m, 256, generator=g).half()                 # a_batches = slots
    idx = torch.tensor([[4, -1, 0], [9, 2, 1]], dtype=torch.int64)
    for lo, hi in ((-1, -1), (1, 4)):
        C0 = torch.full((6, m, 256), 7.0, dtype=torch.float32)
        C = C0.cuda()
        exl3.exl3_mgemm(A.cuda(), B, C, S, None, V, idx.cuda(), None, 3, min_index=lo, max_index=hi)
        ref = oracle.mgemm(A.numpy(), ora, 3, idx.reshape(-1).numpy(), min_index=lo, max_index=hi, C=C0.numpy())
        got = C.cpu().numpy()
        for j in range(6):
            q = oracle.mgemm_matrix(idx.reshape(-1).numpy(), j, 5, lo, hi)
            if q < 0:
                assert np.array_equal(got[j], C0[j].numpy()), (lo, j)
            else:
                assert max_rel(got[j], ref[j]) <= MAX_REL, (lo, j)


@pytest.mark.parametrize("a_mode", ["token", "slot", "broadcast"])
@pytest.mark.parametrize("cdt", [torch.float16, torch.float32])
def test_mgemm_weighted_token_sums(exl3, oracle, synth, a_mode, cdt):
    """Weighted: C[t] = sum over the token's slots of w_j * Y_j in slot order, with skipped slots."""
    T, per, m = 4, 3, 2
    lins, ora = _mats(exl3, synth, 6, 384, 256, 2, 700)
    B, S, V = exl3.mgemm_tables(lins)
    g = torch.Generator().manual_seed(11)
    ab = {"token": T, "slot": T * per, "broadcast": 1}[a_mode]
    A = torch.randn(ab, m, 384, generator=g).half()
    idx = torch.randint(0, 6, (T, per), generator=g)
    idx[1, 2] = -1
    idx[3, :] = -1                                                  # a token with no slot: zero output
    w = (torch.rand(T, per, generator=g) * 2 - 0.5).half()
    C = torch.full((T, m, 256), 3.0, dtype=cdt, device="cuda")
    exl3.exl3_mgemm(A.cuda(), B, C, S, None, V, idx.cuda(), w.cuda(), 2, num_tokens=T)
    ref = oracle.mgemm(A.numpy(), ora, 2, idx.reshape(-1).numpy(), w.reshape(-1).numpy(), num_tokens=T)
    got = C.float().cpu().numpy()
    for t in range(3):
        assert max_rel(got[t], ref[t]) <= MAX_REL, t
    assert (got[3] == 0).all()


def test_mgemm_single_slot_equals_gemm(exl3, synth):
    lins, _ = _mats(exl3, synth, 1, 512, 1024, 4, 800)
    B, S, V = exl3.mgemm_tables(lins)
    A = torch.randn(1, 4, 512, generator=torch.Generator().manual_seed(3)).half().cuda()
    C1 = torch.empty(1, 4, 1024, dtype=torch.float16, device="cuda")
    C2 = torch.empty(4, 1024, dtype=torch.float16, device="cuda")
    exl3.exl3_mgemm(A, B, C1, S, None, V, None, None, 4)
    L = lins[0]
    exl3.exl3_gemm(A[0], L.trellis, C2, L.suh, None, L.svh)
    assert torch.equal(C1[0], C2)


def test_mgemm_composed_moe_layer(exl3, oracle, synth):
    """The exllamav3 BlockSparseMLP decode flow on mgemm: gate and up per slot on the token's x, act, then the
    weighted down sum per token, against the oracle's MoE layer."""
    E, H, I, K, T, k = 8, 256, 256, 3, 3, 2
    from moe_util import make_proj, oracle_proj
    cpu = [[make_proj(H, I, K, 900 + 10 * e), make_proj(H, I, K, 901 + 10 * e), make_proj(I, H, K, 902 + 10 * e)]
           for e in range(E)]
    to = lambda c: exl3.BC_LinearEXL3(c[0].cuda(), c[1].cuda(), c[2].cuda(), K, None, False, True, None)  # noqa
    lins = [[to(cpu[e][p]) for e in range(E)] for p in range(3)]     # the tables hold their addresses: keep them
    tabs = [exl3.mgemm_tables(lins[p]) for p in range(3)]
    g = torch.Generator().manual_seed(12)
    x = torch.randn(T, 1, H, generator=g).half()
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g).half()
    gu = [torch.empty(T * k, 1, I, dtype=torch.float16, device="cuda") for _ in range(2)]
    for p in range(2):
        B, S, V = tabs[p]
        exl3.exl3_mgemm(x.cuda(), B, gu[p], S, None, V, ids.cuda(), None, K, num_tokens=T)
    a = torch.empty_like(gu[0])
    exl3.silu_mul(gu[0], gu[1], a, 0.0)
    out = torch.empty(T, 1, H, dtype=torch.float32, device="cuda")
    B, S, V = tabs[2]
    exl3.exl3_mgemm(a, B, out, S, None, V, ids.cuda(), w.cuda(), K, num_tokens=T)
    orc = [tuple(oracle_proj(oracle, c) for c in cpu[e]) for e in range(E)]
    ref = oracle.moe_layer(x[:, 0].numpy(), orc, ids.numpy(), w.float().numpy(), oracle.ACT_SILU, 0.0)
    assert max_rel(out[:, 0].cpu().numpy(), ref) <= MAX_REL


def test_mgemm_argument_errors(exl3, synth):
    lins, _ = _mats(exl3, synth, 2, 256, 256, 2, 950)
    B, S, V = exl3.mgemm_tables(lins)
    A = torch.zeros(1, 1, 256, dtype=torch.float16, device="cuda")
    C = torch.empty(3, 1, 256, dtype=torch.float16, device="cuda")
    with pytest.raises(exl3.Exl3Error):                              # 3 slots without indices over 2 matrices
        exl3.exl3_mgemm(A, B, C, S, None, V, None, None, 2)
    with pytest.raises(NotImplementedError):
        exl3.exl3_mgemm(A, B, C[:2], S, None, V, None, None, 2, size_n_list=[128, 128])
    with pytest.raises(exl3.Exl3Error):                              # weighted: slots must split over the tokens
        exl3.exl3_mgemm(A, B, C[:2], S, None, V, torch.zeros(3, dtype=torch.int64, device="cuda"),
                        torch.ones(3, dtype=torch.float16, device="cuda"), 2, num_tokens=2)
