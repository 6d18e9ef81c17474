"""Library runtime on the GPU: the fused MoE layer's and the one-row GEMV's bounded waits report a timeout through the
device status word and the next call clears it (the wait is forced to give up from the host with a tiny spin limit, so every kernel
still exits normally), and workspace growth keeps buffers alive that a HIP graph captured earlier still uses."""
import os

import numpy as np
import pytest
import torch

from moe_util import make_experts, max_rel

pytestmark = pytest.mark.gpu
MAX_REL = 2e-3


@pytest.fixture(scope="module")
def layer(exl3, oracle):
    # 48 experts of H = 1024, I = 512 at K = 3; 4 tokens of top-6 = 24 pairs: the one-launch fused decode layer
    tables, orc = make_experts(exl3, oracle, 48, 1024, 512, 3, 3, 4100)
    g = torch.Generator().manual_seed(4101)
    x = torch.randn(4, 1024, generator=g).half()
    logits = torch.randn(4, 48, generator=g)
    ids, w = oracle.route_softmax_topk(logits.numpy(), 6)
    ref = oracle.moe_layer(x.numpy(), orc, ids, w, oracle.ACT_SILU)
    return (tables, x.cuda(), torch.from_numpy(ids.astype(np.int32)).cuda(),
            torch.from_numpy(w.astype(np.float32)).cuda(), ref)


def _call(exl3, layer):
    tables, x, ids, w, _ = layer
    return exl3.moe_forward(x, ids, w, tables)


def test_fused_wait_timeout_is_reported_then_cleared(exl3, oracle, layer):
    lib = exl3._lib
    y = _call(exl3, layer)
    torch.cuda.synchronize()
    assert lib.device_status() == 0
    assert max_rel(y.cpu().numpy(), layer[4]) <= MAX_REL
    print("timeout test: forcing the fused layer's waits to give up (EXL3MI_SPIN_LIMIT=1)", flush=True)
    os.environ["EXL3MI_SPIN_LIMIT"] = "1"
    try:
        for _ in range(4):                  # a down job whose inputs are all in at its first poll does not time out
            _call(exl3, layer)
            torch.cuda.synchronize()
            if lib.device_status():
                break
    finally:
        del os.environ["EXL3MI_SPIN_LIMIT"]
    assert lib.device_status() == 1
    # the next call reports it, zeroes the counters and clears the word
    with pytest.raises(lib.Exl3Error, match="gave up waiting"):
        _call(exl3, layer)
    torch.cuda.synchronize()
    assert lib.device_status() == 0
    # and later calls run normally: the fused layer and a split-K GEMV (both use the counters)
    y = _call(exl3, layer)
    assert max_rel(y.cpu().numpy(), layer[4]) <= MAX_REL
    synth = __import__("importlib").import_module("b70-inference_amd.synth")
    tr, suh, svh = synth.linear(1024, 1024, 4, 4102)
    xs = synth.activations(2, 1024, 4103)
    lin = exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), 4, None, False, True, None)
    yl = lin.run_alloc(xs.cuda(), 1024, True).cpu().numpy()
    ref = oracle.exl3_linear(xs.numpy(), tr.numpy(), suh.numpy(), svh.numpy(), 4, np.float32)
    assert max_rel(yl, ref) <= MAX_REL
    # one row: the tagged split-K exchange, whose words live in the counter buffer that the reset zeroed
    yl1 = lin.run_alloc(xs[:1].cuda(), 1024, True).cpu().numpy()
    assert max_rel(yl1, ref[:1]) <= MAX_REL
    assert lib.device_status() == 0


def test_one_row_gemv_wait_timeout_is_reported_then_cleared(exl3, oracle):
    """The one-row decode GEMV's last k-split waits (bounded) for the other splits' tagged partials. Under a spin
    limit of 1 a wait gives up whenever its first poll misses a word: then the status word is set, the next call
    reports it and zeroes the counter buffer, and later calls are exact again; when every first poll hits, the
    outputs are exact. Either way no stale word survives into a later call."""
    lib = exl3._lib
    synth = __import__("importlib").import_module("b70-inference_amd.synth")
    tr, suh, svh = synth.linear(4096, 5376, 4, 4104)
    xs = synth.activations(1, 4096, 4105)
    lin = exl3.BC_LinearEXL3(tr.cuda(), suh.cuda(), svh.cuda(), 4, None, False, True, None)
    ref = oracle.exl3_linear(xs.numpy(), tr.numpy(), suh.numpy(), svh.numpy(), 4, np.float32)
    xg = xs.cuda()
    print("timeout test: one-row GEMV under EXL3MI_SPIN_LIMIT=1", flush=True)
    os.environ["EXL3MI_SPIN_LIMIT"] = "1"
    try:
        timed_out = False
        for _ in range(8):
            y = lin.run_alloc(xg, 5376, True)
            torch.cuda.synchronize()
            if lib.device_status():
                timed_out = True
                break
            assert max_rel(y.cpu().numpy(), ref) <= MAX_REL
    finally:
        del os.environ["EXL3MI_SPIN_LIMIT"]
    if timed_out:
        with pytest.raises(lib.Exl3Error, match="gave up waiting"):
            lin.run_alloc(xg, 5376, True)
        torch.cuda.synchronize()
        assert lib.device_status() == 0
    for _ in range(3):
        y = lin.run_alloc(xg, 5376, True)
        assert max_rel(y.cpu().numpy(), ref) <= MAX_REL
    assert lib.device_status() == 0


def test_graph_captured_before_growth_replays_on_live_buffers(exl3, oracle, layer):
    """A graph captured before the workspace grows still reads and writes the buffers it captured (growth retires
    them instead of freeing them), and replays give the eager result."""
    lib = exl3._lib
    tables, x, ids, w, ref = layer
    out = torch.empty(4, 1024, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        exl3.moe_forward(x, ids, w, tables, out=out)       # sizes the workspace for this call before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        exl3.moe_forward(x, ids, w, tables, out=out)
    torch.cuda.synchronize()
    # grow the workspace well past anything used so far: the captured buffers are retired, not freed
    lib.reserve_workspace(1 << 31, 1 << 22)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        # eager work on the new buffers between replays
        y = _call(exl3, layer)
        assert torch.equal(y, eager)
    assert max_rel(eager.cpu().numpy(), ref) <= MAX_REL
    del g
    torch.cuda.synchronize()
    lib.release_workspace()
    assert torch.equal(_call(exl3, layer), eager)


# the call refused under capture records nothing, so torch reports the third graph as empty
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_timeout_in_replay_resets_outgrown_counters_and_not_under_capture(exl3, oracle, layer):
    """A lost wait inside a graph replay, on a counter buffer that the workspace has since outgrown: a library call made
    under stream capture reports it and leaves the status word set (a reset recorded into a graph would not run now);
    the next eager call zeroes every counter buffer, the outgrown one included, so a graph captured on it before the
    growth replays the eager result afterwards. The lost wait is forced from the host (a spin limit of 1 captured
    into one graph's launch), so every kernel exits normally."""
    lib = exl3._lib
    tables, x, ids, w, ref = layer
    out_good = torch.empty(4, 1024, dtype=torch.float32, device="cuda")
    out_bad = torch.empty_like(out_good)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        exl3.moe_forward(x, ids, w, tables, out=out_good)  # sizes the workspace before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out_good.clone()
    assert max_rel(eager.cpu().numpy(), ref) <= MAX_REL
    g_good, g_bad = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_good):
        exl3.moe_forward(x, ids, w, tables, out=out_good)
    os.environ["EXL3MI_SPIN_LIMIT"] = "1"
    try:
        with torch.cuda.graph(g_bad):
            exl3.moe_forward(x, ids, w, tables, out=out_bad)
    finally:
        del os.environ["EXL3MI_SPIN_LIMIT"]
    torch.cuda.synchronize()
    lib.reserve_workspace(1 << 31, 1 << 22)                 # both graphs now run on outgrown buffers
    print("timeout test: replaying a graph captured with a spin limit of 1", flush=True)
    for _ in range(4):
        g_bad.replay()
        torch.cuda.synchronize()
        if lib.device_status():
            break
    assert lib.device_status() == 1
    g_cap = torch.cuda.CUDAGraph()
    with pytest.raises(lib.Exl3Error, match="outside stream capture"):
        with torch.cuda.graph(g_cap):
            exl3.moe_forward(x, ids, w, tables, out=out_bad)
    torch.cuda.synchronize()
    assert lib.device_status() == 1
    with pytest.raises(lib.Exl3Error, match="every counter buffer has been reset"):
        lib.reserve_workspace(0, 0)
    torch.cuda.synchronize()
    assert lib.device_status() == 0
    for _ in range(3):
        out_good.zero_()
        g_good.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_good, eager)
        assert torch.equal(_call(exl3, layer), eager)
    assert lib.device_status() == 0
    del g_good, g_bad, g_cap
    torch.cuda.synchronize()
    lib.release_workspace()
