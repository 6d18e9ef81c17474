"""Full-size GPU parity of the benchmarked workloads against the oracle (same seeded bytes on both sides):

  * dense gated MLP 5376 <-> 21504, K = 4, GELU-tanh, 1 / 2 / 4 tokens (every output);
  * MoE prefill layer H = 5120, 160 experts of I = 1536, gate/up K = 2 and down K = 3, 512 tokens routed top-8 by
    softmax over N(0, 1) logits plus a Zipf(1.1) expert bias (the hottest experts hold 200 - 500 rows, i.e. several
    64-row blocks): every row against the oracle, and bit-exact determinism and token-permutation invariance;
  * MoE layer H = 7168, 256 experts of I = 2048 + 1 shared, per-tile K in {1, 2} at 38 / 62 %, 4 decode rows and a
    256-row prefill chunk in one call: every row (with the shared expert) against the oracle, and determinism.

Bar: max|y - r| / max|r| <= 2e-3 (the reference's max_rel, trellis-serve.patch:3889) against the float64-accumulated
oracle; routing ids exact. The oracle decodes and multiplies these sizes in C (oracle/trellis_fast.c)."""
import numpy as np
import pytest
import torch

from moe_util import make_experts, max_rel

pytestmark = pytest.mark.gpu
MAX_REL = 2e-3


def _say(*a):
    print("configs:", *a, flush=True)


def test_dense_gated_mlp_5376_21504_gelu_full_size(exl3, oracle):
    H, I = 5376, 21504
    _say(f"dense gated MLP {H} <-> {I}, K=4, GELU-tanh: building weights")
    tables, orc = make_experts(exl3, oracle, 1, H, I, 4, 4, 2000)
    g, u, d = tables.projs[0][0], tables.projs[1][0], tables.projs[2][0]
    mlp = exl3.BC_GatedMLP(None, None, None, None, None, None, None, 4, False, True, False, True, False, g, u, d, 0.0)
    for M in (1, 2, 4):
        x = torch.randn(M, H, generator=torch.Generator().manual_seed(2100 + M)).half()
        out = torch.empty(1, M, H, dtype=torch.float32, device="cuda")
        mlp.run_bszN(x.cuda().view(1, M, H), out)
        ref = oracle.gated_mlp(x.numpy(), *orc[0], oracle.ACT_GELU_TANH)
        err = max_rel(out.view(M, H).cpu().numpy(), ref)
        _say(f"  M={M} max_rel {err:.2e}")
        assert err <= MAX_REL, (M, err)


def test_moe_prefill_512_tokens_160_experts_zipf_full_size(exl3, oracle):
    E, H, I, M, k = 160, 5120, 1536, 512, 8
    _say(f"MoE prefill {M} tokens, {E} experts {H}/{I}, K 2/3, top-{k} + Zipf bias: building weights")
    tables, orc = make_experts(exl3, oracle, E, H, I, 2, 3, 4400)
    gen = torch.Generator().manual_seed(4401)
    logits = torch.randn(M, E, generator=gen)
    bias = -1.1 * torch.log(torch.randperm(E, generator=gen).float() + 1)
    x = torch.randn(M, H, generator=gen).half()
    ids, w = exl3.route_softmax_topk(logits.cuda(), k, bias.cuda())
    rid, rw = oracle.route_softmax_topk(logits.numpy(), k, bias.numpy())
    assert np.array_equal(ids.cpu().numpy(), rid)
    load = np.bincount(rid.ravel(), minlength=E)
    assert load.max() >= 4 * 64                              # the skew puts several row blocks on the hottest experts
    xc = x.cuda()
    y = exl3.moe_forward(xc, ids, w, tables)
    torch.cuda.synchronize()
    rows = np.arange(M)
    _say(f"  GPU done (max expert load {load.max()} rows); oracle on all {rows.size} rows")
    ref = oracle.moe_layer(x.numpy()[rows], orc, rid[rows], rw[rows], oracle.ACT_SILU)
    err = max_rel(y.cpu().numpy()[rows], ref)
    _say(f"  max_rel {err:.2e}")
    assert err <= MAX_REL, err
    # full size: two calls agree bit for bit, and a token permutation permutes the rows bit for bit
    assert torch.equal(exl3.moe_forward(xc, ids, w, tables), y)
    perm = torch.randperm(M, generator=torch.Generator().manual_seed(4402)).cuda()
    yp = exl3.moe_forward(xc[perm], ids[perm], w[perm], tables)
    assert torch.equal(yp, y[perm])


def test_moe_mixed_1_2_bit_7168_257_experts_decode_and_prefill_rows(exl3, oracle):
    E, H, I, M, k = 256, 7168, 2048, 260, 8
    _say(f"MoE {E}+1 experts {H}/{I}, per-tile K 1/2 at 38/62, {M} rows (4 decode + 256 prefill): building weights")
    tables, orc = make_experts(exl3, oracle, E + 1, H, I, 0, 0, 5000, per_tile=((1, 2), (0.38, 0.62)))
    gen = torch.Generator().manual_seed(5001)
    logits = torch.randn(M, E, generator=gen)
    x = torch.randn(M, H, generator=gen).half()
    ids, w = exl3.route_softmax_topk(logits.cuda(), k)
    rid, rw = oracle.route_softmax_topk(logits.numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    y = exl3.moe_forward(x.cuda(), ids, w, tables, shared=E)
    torch.cuda.synchronize()
    rows = np.arange(M)
    _say(f"  GPU done; oracle on all {rows.size} rows (4 decode + 256 prefill)")
    ref = oracle.moe_layer(x.numpy()[rows], orc[:E], rid[rows], rw[rows], oracle.ACT_SILU, 0.0, orc[E])
    err = max_rel(y.cpu().numpy()[rows], ref)
    _say(f"  max_rel {err:.2e}")
    assert err <= MAX_REL, err
    assert torch.equal(exl3.moe_forward(x.cuda(), ids, w, tables, shared=E), y)
