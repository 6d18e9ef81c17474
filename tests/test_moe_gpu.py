"""GPU parity of the grouped MoE path (routing tables, gate|up + activation epilogue, down, combine, routers, gated
MLP) against the CPU oracle on identical seeded bytes. Bar: max|y - r| / max|r| <= 2e-3 against the oracle's
float64-accumulated layer output (the reference's max_rel, trellis-serve.patch:3889); routing ids exact."""
import numpy as np
import pytest
import torch

from moe_util import make_experts, max_rel

pytestmark = pytest.mark.gpu
MAX_REL = 2e-3


def _ids_w(M, k, E, seed, dup=False, inactive=False):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    if dup and M > 1:
        ids[1, 0] = ids[0, 0]            # same expert in two tokens
    w = torch.rand(M, k, generator=g)
    w = (w / w.sum(1, keepdim=True)).float()
    if inactive:
        ids[0, -1] = -1
    return ids, w


def _run(exl3, oracle, tables, orc, x, ids, w, act=0, limit=0.0, shared=-1, out_dtype=torch.float32):
    out = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables, act, limit, shared, out_dtype=out_dtype)
    ref = oracle.moe_layer(x.numpy(), orc[:tables.E - (1 if shared >= 0 else 0)], ids.numpy(), w.numpy(), act, limit,
                           orc[shared] if shared >= 0 else None)
    return out.float().cpu().numpy(), ref


@pytest.fixture(scope="module")
def small(exl3, oracle):
    return make_experts(exl3, oracle, 12, 256, 256, 3, 3, 500)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 9])
def test_moe_small_silu(exl3, oracle, small, M):
    """Decode batches (the one-launch fused layer at all of these sizes; the multi-kernel path is covered by
    test_moe_fused_and_multi_kernel_paths), an expert shared by two tokens."""
    tables, orc = small
    ids, w = _ids_w(M, 4, 12, 600 + M, dup=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(M)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL


def test_moe_inactive_slots_shared_and_fp16_out(exl3, oracle, small):
    tables, orc = small
    ids, w = _ids_w(3, 3, 11, 701, inactive=True)          # experts 0..10 routed, 11 = shared
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(5)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=11)
    assert max_rel(y, ref) <= MAX_REL
    y16, _ = _run(exl3, oracle, tables, orc, x, ids, w, shared=11, out_dtype=torch.float16)
    assert max_rel(y16, ref) <= MAX_REL


def test_moe_gelu_and_clamp(exl3, oracle, small):
    tables, orc = small
    ids, w = _ids_w(2, 4, 12, 702)
    x = (4 * torch.randn(2, 256, generator=torch.Generator().manual_seed(6))).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, act=1)
    assert max_rel(y, ref) <= MAX_REL
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, act=0, limit=0.5)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M", [1, 2, 4, 7, 8])
def test_moe_fused_and_multi_kernel_paths(exl3, oracle, small, monkeypatch, M):
    """Decode batches take the one-launch fused layer; EXL3MI_NO_FUSED=1 forces the align / gate|up / down launches.
    Both meet the bar, with a shared expert, a repeated expert and an inactive slot."""
    tables, orc = small
    ids, w = _ids_w(M, 3, 11, 710 + M, dup=True, inactive=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(70 + M)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=11)
    assert max_rel(y, ref) <= MAX_REL
    monkeypatch.setenv("EXL3MI_NO_FUSED", "1")
    y2, _ = _run(exl3, oracle, tables, orc, x, ids, w, shared=11)
    assert max_rel(y2, ref) <= MAX_REL


@pytest.mark.parametrize("mr", [1, 2, 4, 8])
@pytest.mark.parametrize("M,k,E,shared", [(8, 4, 4, False), (8, 3, 12, False), (5, 7, 9, False), (7, 3, 10, True)])
def test_moe_multi_kernel_rows_per_item(exl3, oracle, monkeypatch, mr, M, k, E, shared):
    """The multi-launch decode path with every rows-per-item width forced (EXL3MI_MOE_MR; by itself it takes one, two
    or four): experts that take all 8 rows (4 experts top-4), a few rows, a ragged 5-token batch, and a shared expert
    (every token's extra slot: full items at each width beside sparse routed ones), with repeated experts and an
    inactive slot, meet the bar against the oracle; two calls in a row agree bit for bit."""
    tables, orc = make_experts(exl3, oracle, E + shared, 256, 256, 3, 3, 2500 + 10 * E + M)
    ids, w = _ids_w(M, k, E, 2501 + M, dup=True, inactive=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(2502 + M)).half()
    sh = E if shared else -1
    monkeypatch.setenv("EXL3MI_NO_FUSED", "1")
    monkeypatch.setenv("EXL3MI_MOE_MR", str(mr))
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert max_rel(y, ref) <= MAX_REL
    y1, _ = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert np.array_equal(y, y1)


@pytest.mark.parametrize("M,k,E,shared", [(24, 4, 12, False), (17, 3, 11, True), (32, 2, 6, True), (16, 9, 12, False),
                                          (48, 4, 12, True), (64, 2, 8, False)])
def test_moe_items_up_to_64_tokens_and_forced_mfma(exl3, oracle, monkeypatch, M, k, E, shared):
    """Batches of 9 to 64 tokens with uniform K and small experts (and routing dense enough that experts take many
    rows: hot experts in most tokens; past 32 tokens a thin MFMA grid of a few experts) run as GEMV items of up to
    four rows; EXL3MI_MOE_MFMA=1 sends the same batch through the MFMA grouped GEMM. Both meet the bar against the
    oracle, with a shared expert and inactive slots."""
    tables, orc = make_experts(exl3, oracle, E + shared, 256, 256, 3, 3, 2900 + 10 * E + M)
    ids, w = _skewed_ids(M, k, E, 2901 + M)
    ids[0, -1] = -1
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(2902 + M)).half()
    sh = E if shared else -1
    monkeypatch.setenv("EXL3MI_NO_FUSED", "1")
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert max_rel(y, ref) <= MAX_REL
    monkeypatch.setenv("EXL3MI_MOE_MFMA", "1")
    y2, _ = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert max_rel(y2, ref) <= MAX_REL


@pytest.mark.parametrize("M,k,E,shared,no_fused", [(24, 4, 200, False, False), (12, 3, 150, True, True),
                                                   (40, 3, 300, False, False)])
def test_moe_sparse_batches_past_eight_tokens(exl3, oracle, monkeypatch, M, k, E, shared, no_fused):
    """Sparse batches (pairs <= E / 2) of more than 8 tokens that the fused layer does not take (more than 16 tokens,
    or forced off) run as one-row GEMV items on the multi-launch path: with repeated experts, an inactive slot and a
    shared expert (every token's extra slot, a full item per row), they meet the bar against the oracle, and two calls
    in a row agree bit for bit."""
    tables, orc = make_experts(exl3, oracle, E + shared, 256, 256, 3, 3, 2800 + E + M)
    ids, w = _ids_w(M, k, E, 2801 + M, dup=True, inactive=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(2802 + M)).half()
    if no_fused:
        monkeypatch.setenv("EXL3MI_NO_FUSED", "1")
    sh = E if shared else -1
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert max_rel(y, ref) <= MAX_REL
    y1, _ = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert np.array_equal(y, y1)


@pytest.mark.parametrize("mr", [1, 2, 4, 8])
@pytest.mark.parametrize("M,k,E,shared", [(8, 4, 4, False), (16, 7, 16, False), (5, 7, 9, False), (8, 1, 1, False),
                                          (12, 6, 20, True)])
def test_moe_fused_rows_per_item(exl3, oracle, monkeypatch, mr, M, k, E, shared):
    """The fused layer with every rows-per-item width forced (EXL3MI_FUSED_MR; by itself it takes the narrowest
    width whose jobs fit the resident grid): experts that take all 8 rows, 16 tokens over 16 experts, a ragged batch,
    a dense MLP (one expert) and a shared expert beside routed ones, with repeated experts and an inactive slot, meet
    the bar against the oracle; two calls in a row agree bit for bit."""
    tables, orc = make_experts(exl3, oracle, E + shared, 256, 256, 3, 3, 2600 + 10 * E + M)
    ids, w = _ids_w(M, k, E, 2601 + M, dup=True, inactive=k > 1)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(2602 + M)).half()
    sh = E if shared else -1
    monkeypatch.setenv("EXL3MI_FUSED_MR", str(mr))
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert max_rel(y, ref) <= MAX_REL
    y1, _ = _run(exl3, oracle, tables, orc, x, ids, w, shared=sh)
    assert np.array_equal(y, y1)


@pytest.mark.parametrize("M,k,E,Kg,Kd", [(12, 10, 64, 3, 3), (16, 8, 40, 2, 2), (10, 12, 200, 2, 3), (16, 7, 16, 4, 4)])
def test_moe_fused_up_to_16_tokens(exl3, oracle, monkeypatch, M, k, E, Kg, Kd):
    """9 to 16 tokens within 128 pairs take the one-launch layer (items of up to 8 rows, or 2 under sparse routing);
    against the oracle and against the grouped multi-launch path (EXL3MI_NO_FUSED=1: GEMV items up to 16 tokens)."""
    tables, orc = make_experts(exl3, oracle, E, 256, 256, Kg, Kd, 2400 + E + M)
    ids, w = _ids_w(M, k, E, 2401 + M, dup=True, inactive=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(2402 + M)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL
    y1, _ = _run(exl3, oracle, tables, orc, x, ids, w)
    assert np.array_equal(y, y1)
    monkeypatch.setenv("EXL3MI_NO_FUSED", "1")
    y2, _ = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y2, ref) <= MAX_REL


@pytest.mark.parametrize("I,M", [(2048, 1), (2560, 2), (2560, 4)])
def test_moe_fused_split_down_blocks(exl3, oracle, I, M):
    """Wide intermediate (I = 2048: two k splits of the down projection; I = 2560: three, whose staged ranges share
    column blocks of I): each down job waits for just its own blocks of the down input; two calls in a row agree."""
    tables, orc = make_experts(exl3, oracle, 4, 256, I, 3, 3, 1970 + I)
    ids, w = _ids_w(M, 2, 4, 1971 + M, dup=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(1972 + M)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL
    y2, _ = _run(exl3, oracle, tables, orc, x, ids, w)
    assert np.array_equal(y, y2)


def test_moe_fused_counters_reset_between_calls(exl3, small):
    """The fused layer's job ticket and arrival counters are back at zero after every call: alternating batch sizes
    and split counts reproduce the first results bit for bit."""
    tables, _ = small
    xs = {M: torch.randn(M, 256, generator=torch.Generator().manual_seed(90 + M)).half().cuda() for M in (1, 4, 8)}
    rw = {M: _ids_w(M, 4, 12, 720 + M) for M in (1, 4, 8)}
    first = {M: exl3.moe_forward(xs[M], rw[M][0].cuda(), rw[M][1].cuda(), tables) for M in (1, 4, 8)}
    for M in (8, 1, 4, 4, 1, 8):
        again = exl3.moe_forward(xs[M], rw[M][0].cuda(), rw[M][1].cuda(), tables)
        assert torch.equal(again, first[M])


def test_moe_deterministic(exl3, small):
    tables, _ = small
    ids, w = _ids_w(4, 4, 12, 703, dup=True)
    x = torch.randn(4, 256, generator=torch.Generator().manual_seed(7)).half().cuda()
    a = exl3.moe_forward(x, ids.cuda(), w.cuda(), tables)
    b = exl3.moe_forward(x, ids.cuda(), w.cuda(), tables)
    assert torch.equal(a, b)


@pytest.mark.parametrize("Kgu,Kd", [(2, 3), (1, 4), (4, 2), (8, 5)])
def test_moe_per_projection_k(exl3, oracle, Kgu, Kd):
    tables, orc = make_experts(exl3, oracle, 6, 384, 256, Kgu, Kd, 800 + 10 * Kgu + Kd)
    ids, w = _ids_w(2, 3, 6, 801)
    x = torch.randn(2, 384, generator=torch.Generator().manual_seed(8)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("Kgu,Kd", [(2, 3), (3, 4), (1, 3), (6, 8), (4, 3)])
@pytest.mark.parametrize("M", [1, 4, 8])
def test_moe_mixed_bitrate_decode_paths(exl3, oracle, monkeypatch, Kgu, Kd, M):
    """Gate/up and down at different bitrates on the fused decode layer (down one or two bits above gate/up) and on
    the multi-kernel path (every other combination, or forced): both match the oracle, with the shared expert."""
    tables, orc = make_experts(exl3, oracle, 7, 256, 384, Kgu, Kd, 1400 + 10 * Kgu + Kd)
    ids, w = _ids_w(M, 3, 6, 1401 + M)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(1402 + M)).half()
    ref = oracle.moe_layer(x.numpy(), orc[:6], ids.numpy(), w.numpy(), oracle.ACT_SILU, 0.0, orc[6])
    y = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables, shared=6).cpu().numpy()
    assert max_rel(y, ref) <= MAX_REL
    monkeypatch.setenv("EXL3MI_NO_FUSED", "1")
    y2 = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables, shared=6).cpu().numpy()
    assert max_rel(y2, ref) <= MAX_REL


@pytest.mark.parametrize("Ks,probs", [((1, 2), (0.38, 0.62)), ((1, 2, 3, 4, 5, 6, 7, 8), (0.125,) * 8)])
def test_moe_per_tile_k(exl3, oracle, Ks, probs):
    tables, orc = make_experts(exl3, oracle, 5, 256, 384, 0, 0, 900, per_tile=(Ks, probs))
    assert tables.K_gate == 0 and tables.kmaps is not None
    ids, w = _ids_w(3, 2, 5, 901)
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(9)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M,n_logits,bias", [(1, 11, False), (2, 11, True), (4, 11, False), (7, 11, True),
                                               (8, 11, False), (20, 11, True)])
def test_moe_forward_logits_matches_route_then_forward(exl3, small, M, n_logits, bias):
    """The routed entry point returns exactly route_softmax_topk followed by moe_forward: same picks, same weights,
    bit-identical rows (fused decode layer and multi-kernel paths)."""
    tables, _ = small
    g = torch.Generator().manual_seed(1900 + M)
    x = torch.randn(M, 256, generator=g).half().cuda()
    logits = torch.randn(M, n_logits, generator=g).cuda()
    b = (0.3 * torch.randn(n_logits, generator=g)).cuda() if bias else None
    out, ids, w = exl3.moe_forward_logits(x, logits, 3, tables, shared=11, bias=b, return_routing=True)
    rid, rw = exl3.route_softmax_topk(logits, 3, b)
    ref = exl3.moe_forward(x, rid, rw, tables, shared=11)
    assert torch.equal(ids, rid) and torch.equal(w, rw)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("E,k,H,I,biased", [(512, 10, 256, 256, False), (160, 8, 256, 256, True),
                                              (512, 32, 128, 128, True)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5])
def test_moe_forward_logits_in_layer_routing_exact(exl3, oracle, E, k, H, I, biased, M):
    """Routing inside the fused layer (up to 4 tokens; with one row per item each workgroup ranks just its own items'
    tokens) returns the router kernel's picks and weights bit for bit and the same rows as route_softmax_topk +
    moe_forward, at the C3 router shape (512 experts, top-10), a C4-like one (160 experts, top-8, Zipf bias) and
    top-32; 5 tokens take the router kernel."""
    tables, _ = make_experts(exl3, oracle, E, H, I, 2, 2, 2100 + E + k, oracle=False)
    g = torch.Generator().manual_seed(2200 + E + M)
    x = torch.randn(M, H, generator=g).half().cuda()
    logits = (torch.randn(M, E, generator=g) * 2).cuda()
    b = (-1.1 * torch.log(torch.randperm(E, generator=g).float() + 1)).cuda() if biased else None
    out, ids, w = exl3.moe_forward_logits(x, logits, k, tables, bias=b, return_routing=True)
    rid, rw = exl3.route_softmax_topk(logits, k, b)
    assert torch.equal(ids, rid) and torch.equal(w, rw)
    assert torch.equal(out, exl3.moe_forward(x, rid, rw, tables))


@pytest.mark.parametrize("M", [1, 3, 8])
def test_moe_mfma_path_at_decode_sizes(exl3, oracle, monkeypatch, M):
    """The MFMA grouped GEMM at decode batch sizes (per-tile K over wide experts takes it from about 48 active experts
    on; forced here with EXL3MI_MOE_MFMA=1 and the fused layer declined), per-tile K 1 / 2 and a shared expert:
    every expert a single block of at most 16 rows, the oracle's rows to the bar."""
    tables, orc = make_experts(exl3, oracle, 7, 256, 384, 0, 0, 3000 + M, per_tile=((1, 2), (0.38, 0.62)))
    ids, w = _ids_w(M, 3, 6, 3001 + M, dup=True, inactive=True)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(3002 + M)).half()
    monkeypatch.setenv("EXL3MI_FUSED_DECLINE", "1")
    monkeypatch.setenv("EXL3MI_MOE_MFMA", "1")
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=6)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M", [1, 2, 4])
def test_moe_forward_logits_fused_declined(exl3, oracle, small, monkeypatch, M):
    """A batch the fused layer declines (EXL3MI_FUSED_DECLINE=1; by itself it declines those whose gate|up jobs fill
    more than four resident grids) takes the router kernel and the multi-launch path from the routed entry point, at
    sizes that would otherwise rank inside the fused layer: the same picks and weights as the router kernel, the
    same rows as moe_forward on them, and the oracle's rows to the bar, with a shared expert."""
    tables, orc = small
    g = torch.Generator().manual_seed(2350 + M)
    x = torch.randn(M, 256, generator=g).half()
    logits = torch.randn(M, 11, generator=g)
    fused, _, _ = exl3.moe_forward_logits(x.cuda(), logits.cuda(), 3, tables, shared=11, return_routing=True)
    monkeypatch.setenv("EXL3MI_FUSED_DECLINE", "1")
    y, ids, w = exl3.moe_forward_logits(x.cuda(), logits.cuda(), 3, tables, shared=11, return_routing=True)
    rid, rw = exl3.route_softmax_topk(logits.cuda(), 3)
    assert torch.equal(ids, rid) and torch.equal(w, rw)
    assert torch.equal(y, exl3.moe_forward(x.cuda(), rid, rw, tables, shared=11))
    ref = oracle.moe_layer(x.numpy(), orc[:11], rid.cpu().numpy(), rw.cpu().numpy(), oracle.ACT_SILU, 0.0, orc[11])
    assert max_rel(y.cpu().numpy(), ref) <= MAX_REL
    assert max_rel(fused.cpu().numpy(), ref) <= MAX_REL


@pytest.mark.parametrize("M", [1, 2])
def test_moe_forward_logits_in_layer_fp16_and_router_kernel_switch(exl3, small, M, monkeypatch):
    """fp16 outputs of the in-layer routing path, and the same call with the router kernel forced
    (EXL3MI_ROUTER_KERNEL=1): bit-identical rows and picks either way."""
    tables, _ = small
    g = torch.Generator().manual_seed(2300 + M)
    x = torch.randn(M, 256, generator=g).half().cuda()
    logits = torch.randn(M, 11, generator=g).cuda()
    a, ia, wa = exl3.moe_forward_logits(x, logits, 3, tables, shared=11, out_dtype=torch.float16, return_routing=True)
    rid, rw = exl3.route_softmax_topk(logits, 3)
    ref = exl3.moe_forward(x, rid, rw, tables, shared=11, out_dtype=torch.float16)
    assert torch.equal(a, ref) and torch.equal(ia, rid) and torch.equal(wa, rw)
    monkeypatch.setenv("EXL3MI_ROUTER_KERNEL", "1")
    b, ib, wb = exl3.moe_forward_logits(x, logits, 3, tables, shared=11, out_dtype=torch.float16, return_routing=True)
    assert torch.equal(a, b) and torch.equal(ia, ib) and torch.equal(wa, wb)


@pytest.mark.parametrize("M", [1, 4, 12, 37, 160])
def test_moe_packed_tables_same_rows(exl3, small, M):
    """ExpertTables.packed (uniform strides: the decode kernels and the prefill input transform compute expert
    addresses instead of loading them) gives bit-identical rows to the same experts addressed through their pointer
    tables (37 tokens: GEMV items; 160 tokens: the MFMA prefill path)."""
    tables, _ = small
    packed = exl3.ExpertTables.packed(*tables.projs)
    assert packed.layout is not None and list(packed.layout)[9] > 0
    g = torch.Generator().manual_seed(1960 + M)
    x = torch.randn(M, 256, generator=g).half().cuda()
    logits = torch.randn(M, 11, generator=g).cuda()
    a = exl3.moe_forward_logits(x, logits, 3, tables, shared=11)
    b = exl3.moe_forward_logits(x, logits, 3, packed, shared=11)
    assert torch.equal(a, b)


def test_moe_forward_logits_many_experts(exl3, oracle):
    """600 routed experts (the router's 16-register-per-lane variant), top-8: same result as the two calls."""
    tables, _ = make_experts(exl3, oracle, 600, 128, 128, 2, 2, 1950, oracle=False)
    g = torch.Generator().manual_seed(1951)
    x = torch.randn(2, 128, generator=g).half().cuda()
    logits = torch.randn(2, 600, generator=g).cuda()
    out, ids, w = exl3.moe_forward_logits(x, logits, 8, tables, return_routing=True)
    rid, rw = exl3.route_softmax_topk(logits, 8)
    assert torch.equal(ids, rid) and torch.equal(w, rw)
    assert torch.equal(out, exl3.moe_forward(x, rid, rw, tables))


def test_moe_c3_full_size(exl3, oracle):
    """Fine-grained MoE decode layer: H=2048, 512 experts of I=512, K=3, top-10 softmax routing, M = 1, 2, 4."""
    tables, orc = make_experts(exl3, oracle, 512, 2048, 512, 3, 3, 3000)
    for M in (1, 2, 4):
        g = torch.Generator().manual_seed(3100 + M)
        logits = torch.randn(M, 512, generator=g)
        x = torch.randn(M, 2048, generator=g).half()
        ids, w = exl3.route_softmax_topk(logits.cuda(), 10)
        rid, rw = oracle.route_softmax_topk(logits.numpy(), 10)
        assert np.array_equal(ids.cpu().numpy(), rid)
        assert np.abs(w.cpu().numpy() - rw).max() < 1e-6
        y, ref = _run(exl3, oracle, tables, orc, x, ids.cpu(), w.cpu())
        assert max_rel(y, ref) <= MAX_REL, (M, max_rel(y, ref))
        y2 = exl3.moe_forward_logits(x.cuda(), logits.cuda(), 10, tables)
        assert max_rel(y2.cpu().numpy(), ref) <= MAX_REL, M


@pytest.mark.parametrize("M,k,E", [(9, 4, 16), (300, 4, 37), (1500, 4, 37), (2600, 4, 37)])
def test_align_tables(exl3, oracle, M, k, E):
    """Up to 256 pairs take the one-thread-per-pair kernel, more the 1024-thread one: with the pairs held in
    registers and the sorted arrays built in LDS (300 x 4), held but written directly (1500 x 4 = 6000 pairs: the
    LDS copy would not fit 64 KB) and reloaded per phase (2600 x 4 = 10400 pairs, more than 8 per thread)."""
    ids, w = _ids_w(M, k, E, 1000 + M, dup=True, inactive=True)
    counts, ptok, pw, pof = exl3.moe_align(ids.cuda(), w.cuda(), E, shared=-1)
    counts, ptok, pw, pof = (t.cpu().numpy() for t in (counts, ptok, pw, pof))
    ref = oracle.align(ids.numpy(), w.numpy(), E)
    assert np.array_equal(counts, ref["count"])
    flat = ids.numpy().reshape(-1)
    wf = w.numpy().reshape(-1)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    valid_i = np.nonzero(flat >= 0)[0]
    assert (pof[flat < 0] == -1).all()
    pv = pof[valid_i]
    e = flat[valid_i]
    assert ((starts[e] <= pv) & (pv < starts[e] + counts[e])).all()      # grouped by expert
    assert (ptok[pv] == valid_i // k).all() and (pw[pv] == wf[valid_i]).all()
    assert np.unique(pv).size == pv.size == counts.sum()


def test_router_ties_bias_and_sizes(exl3, oracle):
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(7, 160, generator=g)
    logits[0, [5, 40, 99]] = 3.0                 # exact ties: lower index first
    bias = -1.1 * torch.log(torch.arange(1, 161).float())[torch.randperm(160, generator=g)]
    for b in (None, bias):
        ids, w = exl3.route_softmax_topk(logits.cuda(), 8, None if b is None else b.cuda())
        rid, rw = oracle.route_softmax_topk(logits.numpy(), 8, None if b is None else b.numpy())
        assert np.array_equal(ids.cpu().numpy(), rid)
        assert np.abs(w.cpu().numpy() - rw).max() < 1e-6


@pytest.mark.parametrize("M,E,k", [(1, 1, 1), (3, 64, 64 // 2), (4, 100, 7), (4, 512, 10), (2, 1000, 16),
                                   (2, 2048, 8), (1, 4096, 32), (2, 8192, 10)])
def test_router_register_sizes(exl3, oracle, M, E, k):
    """Every values-per-lane variant of the router (E up to 8192, k up to 32), with ties and -inf entries."""
    g = torch.Generator().manual_seed(E * 31 + k)
    logits = torch.randn(M, E, generator=g)
    if E >= 8:
        logits[0, torch.randperm(E, generator=g)[:3]] = 2.5      # exact ties, lower index first
        logits[-1, torch.randperm(E, generator=g)[:2]] = float("-inf")
    ids, w = exl3.route_softmax_topk(logits.cuda(), k, None)
    rid, rw = oracle.route_softmax_topk(logits.numpy(), k, None)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.abs(w.cpu().numpy() - rw).max() < 1e-6


def test_act_mul_ops(exl3, oracle):
    g = torch.Generator().manual_seed(12)
    x = (3 * torch.randn(4, 512, generator=g)).half()
    y = torch.randn(4, 512, generator=g).half()
    for fn, act, lim in ((exl3.silu_mul, 0, 0.0), (exl3.silu_mul, 0, 1.0), (exl3.gelu_mul, 1, 0.0)):
        z = torch.empty_like(x, device="cuda")
        fn(x.cuda(), y.cuda(), z, lim)
        exact = oracle.act_mul(x.numpy(), y.numpy(), act, lim)
        ref = exact.astype(np.float16)
        # within one fp16 ulp of the correctly rounded value (fp32 exp vs the oracle's float64)
        ulp = np.spacing(np.abs(ref)).astype(np.float64)
        assert (np.abs(z.cpu().numpy().astype(np.float64) - ref.astype(np.float64)) <= ulp).all()


def test_gated_mlp_dense(exl3, oracle):
    """Dense gated MLP (GELU-tanh) as the shared-expert path, M = 1, 2, 4."""
    tables, orc = make_experts(exl3, oracle, 1, 512, 1024, 4, 4, 1200)
    g, u, d = tables.projs[0][0], tables.projs[1][0], tables.projs[2][0]
    mlp = exl3.BC_GatedMLP(None, None, None, None, None, None, None, 4, False, True, False, True, False, g, u, d, 0.0)
    for M in (1, 2, 4):
        x = torch.randn(M, 512, generator=torch.Generator().manual_seed(1300 + M)).half()
        out = torch.empty(1, M, 512, dtype=torch.float32, device="cuda")
        mlp.run_bszN(x.cuda().view(1, M, 512), out)
        ref = oracle.gated_mlp(x.numpy(), *orc[0], oracle.ACT_GELU_TANH)
        assert max_rel(out.view(M, 512).cpu().numpy(), ref) <= MAX_REL


def test_block_sparse_mlp_forward(exl3, oracle, small):
    tables, orc = small
    mod = exl3.BlockSparseMLP(tables, 3, has_shared=True)
    g = torch.Generator().manual_seed(14)
    logits = torch.randn(1, 2, 11, generator=g)
    x = torch.randn(1, 2, 256, generator=g).half()
    out = mod.forward(x.cuda(), {"router_logits": logits.cuda()})
    assert out.dtype == torch.float32 and tuple(out.shape) == (1, 2, 256)
    rid, rw = oracle.route_softmax_topk(logits.view(2, 11).numpy(), 3)
    ref = oracle.moe_layer(x.view(2, 256).numpy(), orc[:11], rid, rw, 0, 0.0, orc[11])
    assert max_rel(out.view(2, 256).cpu().numpy(), ref) <= MAX_REL


def test_moe_token_without_active_slots(exl3, oracle, small):
    """A token whose slots are all inactive gets a zero row (and its neighbours are unaffected)."""
    tables, orc = small
    ids, w = _ids_w(3, 3, 12, 1400)
    ids[1, :] = -1
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(15)).half()
    out = torch.full((3, 256), 7.0, device="cuda")
    exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables, out=out)
    ref = oracle.moe_layer(x.numpy(), orc, ids.numpy(), w.numpy(), 0)
    got = out.cpu().numpy()
    assert (got[1] == 0).all()
    assert max_rel(got, ref) <= MAX_REL


def _skewed_ids(M, k, E, seed, hot=(0, 1, 2)):
    """Routing where the `hot` experts appear in most tokens (many rows -> MFMA blocks) and the rest rarely."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.empty(M, k, dtype=torch.int32)
    for t in range(M):
        pool = list(hot) if torch.rand(1, generator=g).item() < 0.85 else []
        rest = [int(e) for e in torch.randperm(E, generator=g) if int(e) not in pool]
        row = (pool + rest)[:k]
        ids[t] = torch.tensor(row, dtype=torch.int32)[torch.randperm(k, generator=g)]
    w = torch.rand(M, k, generator=g)
    return ids, (w / w.sum(1, keepdim=True)).float()


def test_moe_prefill_more_pairs_than_held(exl3, oracle, small):
    """2100 tokens x 4 slots = 8400 pairs: more than the align kernel holds in registers (8 per thread), so it
    reloads the pairs per phase and writes the sorted arrays, the pairs' experts included, from the scatter; every
    row against the oracle."""
    tables, orc = small
    ids, w = _ids_w(2100, 4, 12, 713, dup=True, inactive=True)
    x = torch.randn(2100, 256, generator=torch.Generator().manual_seed(714)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL


def test_moe_prefill_inactive_slots_and_shared(exl3, oracle, small, monkeypatch):
    """Prefill (37 tokens, the MFMA grouped GEMM forced) with a shared expert and inactive slots in several tokens: the
    expert-sorted pairs stop short of tokens x slots (145 of 148 here, not a multiple of 16), so the input transform's
    last row group holds pairs past the valid ones, which it must skip."""
    tables, orc = small
    monkeypatch.setenv("EXL3MI_MOE_MFMA", "1")
    ids, w = _ids_w(37, 3, 11, 711, dup=True, inactive=True)     # experts 0..10 routed, 11 = shared
    ids[5, 1] = -1
    ids[20, 0] = -1
    x = torch.randn(37, 256, generator=torch.Generator().manual_seed(712)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=11)
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("M", [40, 80])
def test_moe_prefill_gemv_and_mfma_paths(exl3, oracle, small, monkeypatch, M):
    """The MFMA grouped GEMM (forced: by itself a batch of up to 128 tokens over these 12 small experts takes GEMV
    items): every expert's rows in blocks of up to 64 rows, hot and cold experts in one call (80 tokens: the hot
    experts cross the 64-row block boundary)."""
    monkeypatch.setenv("EXL3MI_MOE_MFMA", "1")
    tables, orc = small
    ids, w = _skewed_ids(M, 4, 12, 1500 + M)
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(16)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL
    counts = np.bincount(ids.numpy().reshape(-1), minlength=12)
    assert counts.max() > 8 and (counts[counts > 0] <= 8).any()


def test_moe_prefill_per_projection_k_and_gelu(exl3, oracle, monkeypatch):
    monkeypatch.setenv("EXL3MI_MOE_MFMA", "1")                # the MFMA grouped GEMM at 40 tokens
    tables, orc = make_experts(exl3, oracle, 6, 512, 384, 2, 3, 1600)
    ids, w = _skewed_ids(40, 3, 6, 1601, hot=(1, 4))
    x = torch.randn(40, 512, generator=torch.Generator().manual_seed(17)).half()
    for act in (0, 1):
        y, ref = _run(exl3, oracle, tables, orc, x, ids, w, act=act)
        assert max_rel(y, ref) <= MAX_REL


def test_moe_prefill_per_tile_k_shared(exl3, oracle):
    """Per-tile K in {1, 2} (38/62), shared expert on every row (an MFMA expert), routed experts mostly small."""
    tables, orc = make_experts(exl3, oracle, 7, 256, 256, 0, 0, 1700, per_tile=((1, 2), (0.38, 0.62)))
    ids, w = _ids_w(20, 2, 6, 1701)
    x = torch.randn(20, 256, generator=torch.Generator().manual_seed(18)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w, shared=6)
    assert max_rel(y, ref) <= MAX_REL


def test_moe_prefill_per_tile_k_all_bitrates(exl3, oracle):
    """Per-tile K over 1..8 on the MFMA path in all three row classes: the hot experts take about 85 rows each (a
    64-row block plus a 17..32-row block), the rest at most 16; H = 384 leaves the down kernel a half column block."""
    tables, orc = make_experts(exl3, oracle, 10, 384, 256, 0, 0, 1750, per_tile=(tuple(range(1, 9)), (0.125,) * 8))
    ids, w = _skewed_ids(100, 4, 10, 1751)
    counts = np.bincount(ids.numpy().reshape(-1), minlength=10)
    assert counts.max() > 64 and any(16 < c <= 32 for c in counts % 64) and counts.min() <= 16
    x = torch.randn(100, 384, generator=torch.Generator().manual_seed(1752)).half()
    for act in (0, 1):
        y, ref = _run(exl3, oracle, tables, orc, x, ids, w, act=act)
        assert max_rel(y, ref) <= MAX_REL


def test_moe_prefill_per_tile_k_1_2_3(exl3, oracle):
    """Per-tile K in {1, 2, 3} on the MFMA path: most 8-tile steps hold only K <= 3 with some K = 3, which must take
    the run-time decode (the fast path's funnel origins hold for K = 1 and 2 only)."""
    tables, orc = make_experts(exl3, oracle, 6, 256, 256, 0, 0, 1760, per_tile=((1, 2, 3), (0.3, 0.4, 0.3)))
    ids, w = _skewed_ids(60, 3, 6, 1761)
    x = torch.randn(60, 256, generator=torch.Generator().manual_seed(1762)).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL


def test_moe_prefill_many_blocks(exl3, oracle):
    """1100 experts (1200 pairs, more than a thousand row blocks, one expert with 40 rows): the prefill path's
    tables and grids at that size; rows checked against the oracle."""
    E, H, I = 1100, 128, 128
    tables, orc = make_experts(exl3, oracle, E, H, I, 2, 2, 2100)
    M = 600
    g = torch.Generator().manual_seed(2101)
    ids = torch.stack([torch.randperm(E, generator=g)[:2] for _ in range(M)]).to(torch.int32)
    ids[:40, 0] = 7                                      # one expert with 40 rows (a 3-row-group block)
    ids[:40, 1] = torch.where(ids[:40, 1] == 7, torch.full_like(ids[:40, 1], 8), ids[:40, 1])
    w = torch.rand(M, 2, generator=g)
    w = (w / w.sum(1, keepdim=True)).float()
    x = torch.randn(M, H, generator=g).half()
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL


def test_moe_prefill_deterministic_and_token_permutation(exl3, small):
    """Row results do not depend on which other rows share a block: permuting the tokens permutes the output rows
    bit for bit, and two calls agree exactly."""
    tables, _ = small
    ids, w = _skewed_ids(70, 4, 12, 1800)
    x = torch.randn(70, 256, generator=torch.Generator().manual_seed(19)).half()
    perm = torch.randperm(70, generator=torch.Generator().manual_seed(20))
    a = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables)
    b = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables)
    c = exl3.moe_forward(x[perm].cuda(), ids[perm].cuda(), w[perm].cuda(), tables)
    assert torch.equal(a, b)
    assert torch.equal(a[perm.cuda()], c)


def test_moe_c4_shape_rows_vs_oracle(exl3, oracle):
    """C4 shapes (H=5120, I=1536, gate/up K=2, down K=3), 64 tokens over 8 experts with Zipf-skewed softmax routing:
    every row checked against the oracle."""
    tables, orc = make_experts(exl3, oracle, 8, 5120, 1536, 2, 3, 4000)
    g = torch.Generator().manual_seed(4001)
    logits = torch.randn(64, 8, generator=g)
    bias = -1.1 * torch.log(torch.randperm(8, generator=g).float() + 1)
    x = torch.randn(64, 5120, generator=g).half()
    ids, w = exl3.route_softmax_topk(logits.cuda(), 3, bias.cuda())
    rid, rw = oracle.route_softmax_topk(logits.numpy(), 3, bias.numpy())
    assert np.array_equal(ids.cpu().numpy(), rid)
    y, ref = _run(exl3, oracle, tables, orc, x, ids.cpu(), w.cpu())
    assert max_rel(y, ref) <= MAX_REL


@pytest.mark.parametrize("Kgu,Kd", [(2, 3), (4, 4), (6, 6)])
def test_moe_prefill_hot_experts_many_blocks(exl3, oracle, monkeypatch, Kgu, Kd):
    """Hot experts cut into many 64-row blocks of every row class: experts of 520, 300, 257, 256, 130 and 65 rows
    (8 blocks + 8 rows, 4 + 44, 4 + 1, 4, 2 + 2, 1 + 1) beside 40- and 10-row experts, at uniform K with k-permuted
    (K <= 5) and natural-order (K = 6) fragments. Every row against the oracle; the row classes run concurrently on
    three streams or one after another on the caller's stream (EXL3MI_SERIAL_CLASSES=1) with the same rows bit for
    bit; a token permutation permutes the rows bit for bit."""
    E, H, I = 8, 256, 384
    tables, orc = make_experts(exl3, oracle, E, H, I, Kgu, Kd, 2300 + 10 * Kgu)
    loads = [520, 300, 257, 256, 130, 65, 40, 10]
    flat = torch.cat([torch.full((c,), e, dtype=torch.int32) for e, c in enumerate(loads)])
    M = flat.numel() // 2
    ids = torch.stack([flat[:M], flat[M:]], 1)              # sorted halves: a token's two experts differ
    g = torch.Generator().manual_seed(2301)
    ids = ids[torch.randperm(M, generator=g)].contiguous()
    w = torch.rand(M, 2, generator=g)
    w = (w / w.sum(1, keepdim=True)).float()
    x = torch.randn(M, H, generator=g).half()
    print(f"hot experts: K {Kgu}/{Kd}, {M} tokens, loads {loads}", flush=True)
    y, ref = _run(exl3, oracle, tables, orc, x, ids, w)
    assert max_rel(y, ref) <= MAX_REL
    a = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables)
    monkeypatch.setenv("EXL3MI_SERIAL_CLASSES", "1")
    b = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables)
    monkeypatch.delenv("EXL3MI_SERIAL_CLASSES")
    assert torch.equal(a, b)
    perm = torch.randperm(M, generator=g)
    c = exl3.moe_forward(x[perm].cuda(), ids[perm].cuda(), w[perm].cuda(), tables)
    assert torch.equal(a[perm.cuda()], c)
