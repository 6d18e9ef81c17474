"""Edge cases across the entry points on the GPU: empty batches, a batch whose slots are all inactive, a routed
batch larger than the decode path takes (pair lists past 128), and repeated calls with shrinking sizes (library
workspace and counters reused)."""
import pytest
import torch

from moe_util import make_experts, max_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small_layer(exl3, oracle):
    return make_experts(exl3, oracle, 5, 256, 256, 3, 3, 1300)


def test_empty_batches(exl3, small_layer):
    tables, _ = small_layer
    x = torch.empty(0, 256, dtype=torch.float16, device="cuda")
    assert exl3.moe_forward(x, torch.empty(0, 2, dtype=torch.int32, device="cuda"),
                            torch.empty(0, 2, device="cuda"), tables).shape == (0, 256)
    assert exl3.moe_forward_logits(x, torch.empty(0, 4, device="cuda"), 2, tables).shape == (0, 256)
    ids, w = exl3.route_topk(torch.empty(0, 64, device="cuda"), 4, None, "sigmoid")
    assert ids.shape == (0, 4) and w.shape == (0, 4)
    assert exl3.router_logits(x, torch.zeros(256, 64, dtype=torch.float16, device="cuda")).shape == (0, 64)
    g = tables.projs[0][0]
    assert g.run_alloc(x, g.out_features, True).shape == (0, 256)
    tr, suh, svh, sonb, b, K = exl3.fuse_linears([tables.projs[0][0], tables.projs[1][0]])
    assert exl3.linear(x, tr, suh, svh, sonb, b, K).shape == (0, 512)


@pytest.mark.parametrize("M", [1, 6, 40])
def test_all_slots_inactive(exl3, oracle, small_layer, M):
    """Every slot of every token inactive: zero rows; with the shared expert: exactly the shared expert."""
    tables, orc = small_layer
    x = torch.randn(M, 256, generator=torch.Generator().manual_seed(M)).half()
    ids = torch.full((M, 3), -1, dtype=torch.int32)
    w = torch.rand(M, 3)
    y = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables)
    assert torch.count_nonzero(y) == 0
    ys = exl3.moe_forward(x.cuda(), ids.cuda(), w.cuda(), tables, shared=4)
    ref = oracle.moe_layer(x.numpy(), orc[:4], ids.numpy(), w.numpy(), oracle.ACT_SILU, 0.0, orc[4])
    assert max_rel(ys.cpu().numpy(), ref) <= 2e-3


def test_shrinking_then_growing_batches(exl3, oracle, small_layer):
    """Batch sizes across the decode / multi-kernel / MFMA paths in a row (shared workspace and counters)."""
    tables, orc = small_layer
    g = torch.Generator().manual_seed(77)
    for M in (64, 3, 17, 1, 130, 8, 2):
        x = torch.randn(M, 256, generator=g).half()
        logits = torch.randn(M, 4, generator=g)
        y, ids, w = exl3.moe_forward_logits(x.cuda(), logits.cuda(), 2, tables, shared=4, return_routing=True)
        ref = oracle.moe_layer(x.numpy(), orc[:4], ids.cpu().numpy(), w.cpu().numpy(), oracle.ACT_SILU, 0.0, orc[4])
        assert max_rel(y.cpu().numpy(), ref) <= 2e-3, M
