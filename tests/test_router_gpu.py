"""GPU parity of the routers: scored top-k (softmax / sigmoid / sqrt-softplus, bias, renormalisation, scaling) and the
router GEMV from hidden states (both weight layouts), against the CPU oracle on the same seeded inputs.

Bars: routing ids identical; weights within 1e-5 relative (fp32 scores against the oracle's float64 weights); fp32
logits within 1e-5 of max |logit| (fp32 sums in a different order); fp16-rounded logits within that plus one fp16 ulp
(a sum near a rounding boundary may round the other way).
"""
import numpy as np
import pytest
import torch

from moe_util import make_experts, max_rel

pytestmark = pytest.mark.gpu


def _close16(y, ref):
    """fp16-rounded logits: |y - ref| <= 1e-5 max|ref| + one fp16 ulp of ref."""
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return bool((np.abs(y.astype(np.float64) - ref) <= 1e-5 * np.abs(ref).max() + ulp).all())


def _logits(M, E, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, E, generator=g) * scale, torch.randn(E, generator=g) * 0.5


@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrt_softplus"])
@pytest.mark.parametrize("E,k", [(64, 1), (160, 8), (512, 10), (1000, 32)])
@pytest.mark.parametrize("bias_mode", ["none", "both", "select"])
def test_route_topk_matches_oracle(exl3, oracle, score, E, k, bias_mode):
    M = 37
    logits, bias = _logits(M, E, 100 + E + k + len(score))
    b = None if bias_mode == "none" else bias
    for renorm, scaling in ((True, 1.0), (True, 2.5), (False, 1.0)):
        ids, w = exl3.route_topk(logits.cuda(), k, None if b is None else b.cuda(), score, renorm, scaling,
                                 bias_select_only=bias_mode == "select")
        rid, rw = oracle.route_topk(logits.numpy(), k, None if b is None else b.numpy(), score, renorm, scaling,
                                    bias_select_only=bias_mode == "select")
        assert np.array_equal(ids.cpu().numpy(), rid), (renorm, scaling)
        assert np.abs(w.cpu().numpy() - rw).max() <= 1e-5 * max(1.0, float(np.abs(rw).max())), (renorm, scaling)


@pytest.mark.parametrize("E,k", [(512, 10), (1000, 32), (4096, 32), (8192, 24)])
def test_route_topk_picks_crowded_in_few_lanes(exl3, oracle, E, k):
    """The top picks sit in one or two wave lanes (indices l + 64 v), with exact ties inside a lane and across
    lanes: a lane is picked many times in a row, so its cache of best keys empties and refills repeatedly."""
    g = torch.Generator().manual_seed(E + k)
    logits = torch.randn(4, E, generator=g)
    V = (E + 63) // 64
    lane_a = torch.arange(5, E, 64)[: V]                     # lane 5, every value slot
    lane_b = torch.arange(40, E, 64)[: V]
    logits[0, lane_a] = 10.0 + torch.arange(len(lane_a)).float() % 3          # ties inside the lane
    logits[1, lane_a] = 9.0
    logits[1, lane_b] = 9.0                                                    # ties across two lanes
    logits[2, lane_b] = 8.0 - torch.arange(len(lane_b)).float() * 0.25
    logits[2, lane_a[: k // 2]] = 8.0                                          # ties with lane b's best
    logits[3, lane_a] = float("-inf")
    logits[3, lane_b[:3]] = float("-inf")
    for score in ("softmax", "sigmoid"):
        ids, w = exl3.route_topk(logits.cuda(), k, None, score)
        rid, rw = oracle.route_topk(logits.numpy(), k, None, score)
        assert np.array_equal(ids.cpu().numpy(), rid), score
        assert np.abs(w.cpu().numpy() - rw).max() <= 1e-6, score


def test_route_softmax_topk_unchanged_by_generalisation(exl3):
    """exl3_route_softmax_topk is route_topk(softmax, bias ranks and weights, renormalised): bit-identical results."""
    logits, bias = _logits(20, 512, 7)
    a = exl3.route_softmax_topk(logits.cuda(), 10, bias.cuda())
    b = exl3.route_topk(logits.cuda(), 10, bias.cuda(), "softmax")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_route_topk_ties_and_small_rows(exl3, oracle):
    """Exact ties rank to the lower index; k == E picks every expert."""
    logits = torch.zeros(3, 32)
    logits[1, ::3] = 1.0
    logits[2] = torch.arange(32).float().flip(0) % 5
    for score in ("softmax", "sigmoid", "sqrt_softplus"):
        ids, w = exl3.route_topk(logits.cuda(), 32, None, score)
        rid, rw = oracle.route_topk(logits.numpy(), 32, None, score)
        assert np.array_equal(ids.cpu().numpy(), rid)
        assert np.abs(w.cpu().numpy() - rw).max() <= 1e-6


@pytest.mark.parametrize("score", ["sigmoid", "sqrt_softplus"])
@pytest.mark.parametrize("E,k", [(64, 1), (160, 6), (256, 8), (1000, 8)])
@pytest.mark.parametrize("terms", ["mul", "res", "both"])
def test_route_adjusted_matches_oracle(exl3, oracle, score, E, k, terms):
    """Residency-adjusted ranking s * mul + bias + max(res, -1e30): picks identical to the oracle, weights from s."""
    M = 9
    logits, bias = _logits(M, E, 300 + E + k)
    g = torch.Generator().manual_seed(400 + E)
    mul = (0.5 + 1.5 * torch.rand(E, generator=g)) if terms in ("mul", "both") else None
    res = None
    if terms in ("res", "both"):
        u = torch.rand(E, generator=g)
        res = torch.where(u < 0.2, torch.tensor(float("-inf")), torch.where(u < 0.5, torch.tensor(-0.75),
                                                                             torch.tensor(0.0)))
    for scaling in (1.0, 2.5):
        ids, w = exl3.route_adjusted(logits.cuda(), k, bias.cuda(), None if mul is None else mul.cuda(),
                                     None if res is None else res.cuda(), score, True, scaling)
        rid, rw = oracle.route_topk(logits.numpy(), k, bias.numpy(), score, True, scaling,
                                    mul=None if mul is None else mul.numpy(), res=None if res is None else res.numpy())
        assert np.array_equal(ids.cpu().numpy(), rid), scaling
        assert np.abs(w.cpu().numpy() - rw).max() <= 1e-5 * max(1.0, float(np.abs(rw).max()))


def test_moe_route_in_place(exl3, oracle):
    """The reference op's signature: int64 ids / want written in place, want = the plain sqrt-softplus top-k."""
    M, E, k = 5, 256, 8
    logits, bias = _logits(M, E, 77)
    res = torch.zeros(E)
    res[::4] = -1.0
    ids = torch.empty(M, k, dtype=torch.int64, device="cuda")
    w = torch.empty(M, k, dtype=torch.float32, device="cuda")
    want = torch.empty(M, k, dtype=torch.int64, device="cuda")
    exl3.moe_route(logits.cuda(), bias.cuda(), res.cuda(), ids, w, want, 2.0)
    rid, rw = oracle.route_topk(logits.numpy(), k, bias.numpy(), "sqrt_softplus", True, 2.0, res=res.numpy())
    pid, _ = oracle.route_topk(logits.numpy(), k, bias.numpy(), "sqrt_softplus", True, 2.0)
    assert np.array_equal(ids.cpu().numpy(), rid) and np.array_equal(want.cpu().numpy(), pid)
    assert np.abs(w.cpu().numpy() - rw).max() <= 1e-5 * 2.0


@pytest.mark.parametrize("E,k,S,boost", [(64, 4, 2, 0.5), (256, 8, 4, 0.25), (1000, 6, 3, 1.0), (256, 8, 4, 0.0)])
@pytest.mark.parametrize("with_mul", [False, True])
def test_route_block_matches_oracle(exl3, oracle, E, k, S, boost, with_mul):
    """Verify-block routing: rows of a block in order, earlier rows' experts boosted; picks identical to the oracle."""
    M = 4 * S
    logits, bias = _logits(M, E, 500 + E + S)
    mul = (0.5 + torch.rand(E, generator=torch.Generator().manual_seed(E))) if with_mul else None
    ids, w = exl3.route_block(logits.cuda(), k, bias.cuda(), None if mul is None else mul.cuda(), S, boost, 1.5)
    rid, rw = oracle.route_block(logits.numpy(), k, bias.numpy(), None if mul is None else mul.numpy(), S, boost, 1.5)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.abs(w.cpu().numpy() - rw).max() <= 1e-5 * 1.5


@pytest.mark.parametrize("S,boost,with_res", [(1, 0.0, True), (2, 0.5, False), (2, 0.5, True)])
def test_route_fused_two_layers(exl3, oracle, S, boost, with_res):
    """route_fused with the reference op's signature: logits of this layer's and the next layer's gates in one buffer,
    this layer's picks (residency or block boost), the plain picks, and the next layer's picks."""
    g = torch.Generator().manual_seed(600 + S)
    R, H, E0, E1, k = 4, 512, 256, 160, 8
    x = torch.randn(R, H, generator=g).half()
    w0 = (torch.randn(E0, H, generator=g) / H ** 0.5).half()
    w1 = (torch.randn(E1, H, generator=g) / H ** 0.5).half()
    b0, b1 = torch.randn(E0, generator=g) * 0.1, torch.randn(E1, generator=g) * 0.1
    m0, m1 = 1 + torch.rand(E0, generator=g), 1 + torch.rand(E1, generator=g)
    res = torch.where(torch.rand(E0, generator=g) < 0.3, torch.tensor(-0.5), torch.tensor(0.0)) if with_res else None
    dev = lambda t: None if t is None else t.cuda()  # noqa: E731
    ids0 = torch.empty(R, k, dtype=torch.int64, device="cuda")
    want0 = torch.empty(R, k, dtype=torch.int64, device="cuda")
    ids1 = torch.empty(R, k, dtype=torch.int64, device="cuda")
    w0o = torch.empty(R, k, device="cuda")
    w1o = torch.empty(R, k, device="cuda")
    logits = torch.empty(R * (E0 + E1), device="cuda")
    exl3.route_fused(x.cuda(), w0.cuda(), w1.cuda(), b0.cuda(), b1.cuda(), dev(res), ids0, w0o, want0, ids1, w1o,
                     logits, 1.5, 2.0, m0.cuda(), m1.cuda(), S, boost)
    lg = logits.view(R, E0 + E1).cpu().numpy()
    ref0 = oracle.router_logits(x.numpy(), w0.numpy(), "eh")
    ref1 = oracle.router_logits(x.numpy(), w1.numpy(), "eh")
    assert np.abs(lg[:, :E0] - ref0).max() <= 1e-5 * np.abs(ref0).max()
    assert np.abs(lg[:, E0:] - ref1).max() <= 1e-5 * np.abs(ref1).max()
    # picks from the GPU's own logits (a logit one ulp from the oracle's could reorder a near-tie)
    l0, l1 = lg[:, :E0].copy(), lg[:, E0:].copy()
    if S > 1 and boost > 0 and res is None:
        rid0, rw0 = oracle.route_block(l0, k, b0.numpy(), m0.numpy(), S, boost, 1.5)
        rid1, rw1 = oracle.route_block(l1, k, b1.numpy(), m1.numpy(), S, boost, 2.0)
    else:
        rid0, rw0 = oracle.route_topk(l0, k, b0.numpy(), "sqrt_softplus", True, 1.5, mul=m0.numpy(),
                                      res=None if res is None else res.numpy())
        if S > 1 and boost > 0:
            rid1, rw1 = oracle.route_block(l1, k, b1.numpy(), m1.numpy(), S, boost, 2.0)
        else:
            rid1, rw1 = oracle.route_topk(l1, k, b1.numpy(), "sqrt_softplus", True, 2.0, mul=m1.numpy())
    pid, _ = oracle.route_topk(l0, k, b0.numpy(), "sqrt_softplus", True, 1.5)
    assert np.array_equal(ids0.cpu().numpy(), rid0) and np.array_equal(want0.cpu().numpy(), pid)
    assert np.array_equal(ids1.cpu().numpy(), rid1)
    assert np.abs(w0o.cpu().numpy() - rw0).max() <= 1e-5 * 1.5 and np.abs(w1o.cpu().numpy() - rw1).max() <= 2e-5


@pytest.mark.parametrize("layout", ["he", "eh"])
@pytest.mark.parametrize("H,E", [(128, 72), (2048, 512), (5120, 160), (7168, 256)])
@pytest.mark.parametrize("M", [1, 3, 4, 9, 33])
def test_router_logits_matches_oracle(exl3, oracle, layout, H, E, M):
    g = torch.Generator().manual_seed(H + E + M)
    x = torch.randn(M, H, generator=g).half()
    W = (torch.randn(H, E, generator=g) / H ** 0.5).half()
    Wl = W if layout == "he" else W.T.contiguous()
    for r16 in (False, True):
        y = exl3.router_logits(x.cuda(), Wl.cuda(), E, layout, r16).cpu().numpy()
        ref = oracle.router_logits(x.numpy(), Wl.numpy(), layout, r16)
        if r16:
            assert _close16(y, ref)
        else:
            assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


def test_router_logits_strided_gate_columns(exl3, oracle):
    """gate[:, :E] of a wider (padded) gate tensor, as routing_ds3_nogroup passes it."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 1024, generator=g).half()
    Wp = (torch.randn(1024, 264, generator=g) / 32).half()
    y = exl3.router_logits(x.cuda(), Wp.cuda()[:, :256], 256, "he").cpu().numpy()
    ref = oracle.router_logits(x.numpy(), Wp[:, :256].contiguous().numpy(), "he")
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


def test_routing_ds3_nogroup_in_place(exl3, oracle):
    """The reference op's signature and in-place outputs (glm/xpu/glm_xpu/ops.py:177-193)."""
    g = torch.Generator().manual_seed(9)
    M, H, E, k = 6, 2048, 256, 8
    hidden = torch.randn(M, H, generator=g).half()
    gate = (torch.randn(H, E + 8, generator=g) / H ** 0.5).half()
    bias = torch.randn(E, generator=g) * 0.1
    scores = torch.empty(M, E, dtype=torch.float32, device="cuda")
    ti = torch.empty(M, k, dtype=torch.int64, device="cuda")
    tw = torch.empty(M, k, dtype=torch.float32, device="cuda")
    exl3.routing_ds3_nogroup(hidden.cuda(), gate.cuda(), scores, bias.cuda(), ti, tw, 2.5, None, 0, None, None)
    lg = oracle.router_logits(hidden.numpy(), gate[:, :E].contiguous().numpy(), "he", True)
    rid, rw = oracle.route_topk(lg, k, bias.numpy(), "sigmoid", True, 2.5)
    assert _close16(scores.cpu().numpy(), lg)
    # ids can only differ where a logit sits one ulp apart from the oracle's: recompute from the GPU's own scores
    rid2, rw2 = oracle.route_topk(scores.cpu().numpy(), k, bias.numpy(), "sigmoid", True, 2.5)
    assert np.array_equal(ti.cpu().numpy(), rid2)
    assert np.abs(tw.cpu().numpy() - rw2).max() <= 1e-5
    assert (rid == rid2).mean() > 0.9
    with pytest.raises(NotImplementedError):
        exl3.routing_ds3_nogroup(hidden.cuda(), gate.cuda(), scores, None, ti, tw, 1.0, None, 1, None, None)


@pytest.mark.parametrize("score,layout", [("sigmoid", "he"), ("sqrt_softplus", "eh"), ("softmax", "he")])
def test_block_sparse_mlp_router_weight_and_scoring(exl3, oracle, score, layout):
    """BlockSparseMLP from hidden states: native router GEMV, scored top-k, grouped experts, shared expert."""
    E, H, I, k = 8, 256, 256, 2
    tables, orc = make_experts(exl3, oracle, E + 1, H, I, 3, 3, 900)
    g = torch.Generator().manual_seed(901)
    W = (torch.randn(H, E, generator=g) / 16).half()
    bias = torch.randn(E, generator=g) * 0.3
    Wl = W if layout == "he" else W.T.contiguous()
    mlp = exl3.BlockSparseMLP(tables, k, has_shared=True, router_weight=Wl.cuda(), selection_bias=bias.cuda(),
                              scoring=score, routed_scaling=1.5 if score != "softmax" else 1.0,
                              bias_select_only=score == "softmax", router_layout=layout)
    for M in (3, 12):
        x = torch.randn(M, H, generator=g).half()
        y = mlp.forward(x.cuda()).cpu().numpy()
        lg = exl3.router_logits(x.cuda(), Wl.cuda(), E, layout).cpu().numpy()
        rid, rw = oracle.route_topk(lg, k, bias.numpy(), score, True, mlp.routed_scaling,
                                    bias_select_only=score == "softmax")
        ref = oracle.moe_layer(x.numpy(), orc[:E], rid, rw, oracle.ACT_SILU, 0.0, orc[E])
        assert max_rel(y, ref) <= 2e-3, M
