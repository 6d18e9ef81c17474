"""Expert records and the record store (host side), the reference's expert blob unpacked (against the oracle's
restatement of its packer), and (GPU) the arena-packed experts giving the same layer outputs as separately allocated
ones."""
import importlib
import math

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O

blob = importlib.import_module("b70-inference_amd.blob")
synth = importlib.import_module("b70-inference_amd.synth")


def _expert(H, I, Kgu, Kd, seed):
    g = synth.linear(H, I, Kgu, seed)
    u = synth.linear(H, I, Kgu, seed + 1)
    d = synth.linear(I, H, Kd, seed + 2)
    return [{"trellis": t, "suh": su, "svh": sv} for t, su, sv in (g, u, d)]


def test_reference_planar4_is_a_permutation_and_identity_for_even_k():
    """The reference's own check (pack_store.py:58) and its K = 4 note (moe_offload.py:71-73)."""
    for K in (2, 3, 4, 5, 6, 7, 8):
        idx = np.arange(2 * 8 * 8 * K, dtype=np.uint32)
        tr32 = idx.view(np.int16).reshape(2, 8, 16 * K)
        w = O.planar4_words(tr32, K)
        assert np.array_equal(np.sort(w), idx)
        if K in (2, 4, 8):
            assert np.array_equal(w, idx)
        else:
            assert not np.array_equal(w, idx)


def _planar4_by_loops(words, K):
    """PLANAR4 as the reference's kernel comment states it (exl3_moe.n128.sycl:8-11): within every k-row the tiles
    are grouped by 4 along n, and word (tile t, period g, plane i) of a group, at [t][D g + i] in tile order, is
    stored at [i][t][g]. words: uint32 [rows, tiles, 8K] in tile order. Built element by element."""
    rows, tiles, W = words.shape
    D = K // math.gcd(K, 32)
    G = W // D
    out = np.empty(words.size, dtype=np.uint32)
    pos = 0
    for r in range(rows):
        for grp in range(tiles // 4):
            for i in range(D):
                for t in range(4):
                    for g in range(G):
                        out[pos] = words[r, 4 * grp + t, D * g + i]
                        pos += 1
    return out


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
def test_planar4_matches_the_loop_built_index_map(K):
    """The oracle's reshape/transpose statement of PLANAR4 equals the element loop for every K (a transposed
    [tile][plane] order or swapped period/plane index fails: odd K has D = K planes of 8 periods)."""
    rows, tiles = 3, 8
    idx = np.arange(rows * tiles * 8 * K, dtype=np.uint32)
    tr = idx.view(np.int16).reshape(rows, tiles, 16 * K)
    assert np.array_equal(O.planar4_words(tr, K), _planar4_by_loops(idx.reshape(rows, tiles, 8 * K), K))
    if K == 3:
        # spot values: group 0 of row 0 starts with plane 0 of tiles 0..3 (words 0, 3, 6, ... of tile 0)
        w = O.planar4_words(tr, K)
        assert list(w[:9]) == [0, 3, 6, 9, 12, 15, 18, 21, 24]
        assert w[8] == 24 and w[8 * 4] == 1 and w[8 * 4 * 3 - 1] == 4 * 24 - 1


@pytest.mark.parametrize("K", [2, 3, 4, 5, 6])
def test_unpack_reference_blob_round_trip(K):
    H, I = 256, 128
    gate, up, down = _expert(H, I, K, K, 700 + K)
    b = O.reference_blob(*[{k: v.numpy() for k, v in p.items()} for p in (gate, up, down)], K)
    assert b.size == O.reference_geom_bytes(H, I, K)
    g2, u2, d2 = blob.unpack_reference_blob(torch.from_numpy(b), H, I, K)
    for a, r in ((gate, g2), (up, u2), (down, d2)):
        for kind in ("trellis", "suh", "svh"):
            assert torch.equal(a[kind], r[kind]), kind


def test_record_pack_views_and_arena_layout():
    H, I, Kgu, Kd = 256, 384, 2, 3
    geom = blob.RecordGeom(H, I, Kgu, Kd)
    assert geom.bytes % 4096 == 0
    offs = sorted(v[0] for v in geom.sections.values())
    assert offs[0] == 0 and all(o % 256 == 0 for o in offs)
    experts = [_expert(H, I, Kgu, Kd, 800 + 10 * e) for e in range(3)]
    arena = blob.ExpertArena(3, geom, device="cpu")
    for e, ex in enumerate(experts):
        arena.put(e, *ex)
    for e, views in enumerate(arena.experts()):
        for src, v in zip(experts[e], views):
            assert torch.equal(src["trellis"], v.trellis)
            assert torch.equal(src["suh"], v.suh) and torch.equal(src["svh"], v.svh)
    tabs = arena.tables()
    assert tabs.layout is not None                       # uniform strides: base + e * record bytes
    assert list(tabs.layout)[9:] == [geom.bytes] * 9
    assert (tabs.K_gate, tabs.K_up, tabs.K_down) == (Kgu, Kgu, Kd)
    with pytest.raises(RuntimeError):
        blob.pack_expert(experts[0][0], experts[0][1], experts[0][0], geom)    # down shape wrong


def test_store_write_verify_load(tmp_path):
    H, I = 256, 128
    g1, g2 = blob.RecordGeom(H, I, 3), blob.RecordGeom(H, I, 2, 3)
    l1 = [_expert(H, I, 3, 3, 900 + 10 * e) for e in range(4)]
    l2 = [_expert(H, I, 2, 3, 950 + 10 * e) for e in range(2)]
    path = str(tmp_path / "experts")
    man = blob.write_store(path, [(g1, l1), (g2, l2)])
    assert man["layers"][1]["offset"] == 4 * g1.bytes
    assert blob.verify_store(path) == []
    arena = blob.load_layer(path, 1, device="cpu")
    views = arena.experts()
    for e in range(2):
        for src, v in zip(l2[e], views[e]):
            assert torch.equal(src["trellis"], v.trellis)
    # a flipped byte in layer 0, expert 2 is found, and loading that layer refuses
    with open(path + ".bin", "r+b") as f:
        f.seek(2 * g1.bytes + 1000)
        c = f.read(1)
        f.seek(2 * g1.bytes + 1000)
        f.write(bytes([c[0] ^ 1]))
    assert blob.verify_store(path) == [(0, 2)]
    with pytest.raises(RuntimeError):
        blob.load_layer(path, 0, device="cpu")


@pytest.mark.gpu
@pytest.mark.parametrize("M", [3, 40])
def test_arena_experts_same_outputs(exl3, M):
    """Arena-packed experts (uniform-stride tables) and separately allocated copies give bit-identical layers, within
    the tolerance of the oracle's layer."""
    E, H, I = 6, 256, 256
    geom = blob.RecordGeom(H, I, 3)
    experts = [_expert(H, I, 3, 3, 1000 + 10 * e) for e in range(E)]
    arena = blob.ExpertArena(E, geom, device="cuda")
    for e, ex in enumerate(experts):
        arena.put(e, *ex)
    t_arena = arena.tables()
    assert t_arena.layout is not None

    def lin(p):
        return exl3.BC_LinearEXL3(p["trellis"].cuda(), p["suh"].cuda(), p["svh"].cuda(), 3, None, False, True, None)

    t_sep = exl3.ExpertTables([lin(x[0]) for x in experts], [lin(x[1]) for x in experts],
                              [lin(x[2]) for x in experts])
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, H, generator=g).half().cuda()
    logits = torch.randn(M, E, generator=g).cuda()
    a = exl3.moe_forward_logits(x, logits, 2, t_arena)
    b = exl3.moe_forward_logits(x, logits, 2, t_sep)
    assert torch.equal(a, b)
    # and the arena layer against the oracle's layer on the same experts and routing
    rid, rw = O.route_softmax_topk(logits.cpu().numpy(), 2)
    orc = [tuple(O.Proj(p["suh"].numpy(), p["svh"].numpy(), trellis=p["trellis"].numpy(), K=3) for p in ex)
           for ex in experts]
    ref = O.moe_layer(x.cpu().numpy(), orc, rid, rw, O.ACT_SILU)
    err = float(np.abs(a.cpu().numpy() - ref).max() / np.abs(ref).max())
    assert err <= 2e-3, err


# decode paths of the layer by batch shape: (tokens, top-k, experts) -> the one-launch fused layer (<= 16 tokens, <= 128
# pairs), the multi-kernel decode GEMVs (<= 8 tokens, more than 128 pairs), the MFMA grouped GEMM (160 tokens)
BLOB_PATHS = {"fused": (3, 2, 6), "gemv": (8, 17, 20), "mfma": (160, 2, 6)}


@pytest.mark.gpu
@pytest.mark.parametrize("K", [2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("HI", [(256, 384), (384, 256)])
@pytest.mark.parametrize("path", list(BLOB_PATHS))
def test_moe_forward_blobs_on_reference_blobs(exl3, K, HI, path):
    """The reference's blob-pointer op on blobs exactly as the reference packs them (pack_expert / planar4, restated in
    the oracle and pinned by the element-loop index map above; PLANAR4 differs from tile order at K = 3, 5, 6, 7), one
    device blob per expert, read in place: the layer equals exl3_moe_forward on separately allocated tensors bit for
    bit and the oracle's layer to 2e-3, on each decode path, with H != I both ways (so a swapped H / I in the blob
    offsets fails). The blobs are not modified by the call."""
    H, I = HI
    M, topk, E = BLOB_PATHS[path]
    experts = [_expert(H, I, K, K, 1200 + 10 * e + K) for e in range(E)]
    host = [O.reference_blob(*[{k: v.numpy() for k, v in p.items()} for p in ex], K) for ex in experts]
    blobs = [torch.from_numpy(b).cuda() for b in host]
    ptrs = torch.tensor([b.data_ptr() for b in blobs], dtype=torch.int64, device="cuda")
    g = torch.Generator().manual_seed(1300 + 10 * M + K)
    x = torch.randn(M, H, generator=g).half()
    logits = torch.randn(M, E, generator=g)
    rid, rw = O.route_softmax_topk(logits.numpy(), topk)
    ids = torch.from_numpy(rid.astype(np.int32)).cuda()
    w = torch.from_numpy(rw.astype(np.float32)).cuda()
    print(f"blob op: K={K} H={H} I={I} {path} M={M} top-{topk} of {E}", flush=True)
    y = exl3.moe_forward_blobs(x.cuda(), ids, w, ptrs, I, K, E, out_dtype=torch.float32)

    def lin(p):
        return exl3.BC_LinearEXL3(p["trellis"].cuda(), p["suh"].cuda(), p["svh"].cuda(), K, None, False, True, None)

    t_sep = exl3.ExpertTables([lin(ex[0]) for ex in experts], [lin(ex[1]) for ex in experts],
                              [lin(ex[2]) for ex in experts])
    assert torch.equal(y, exl3.moe_forward(x.cuda(), ids, w, t_sep))
    orc = [tuple(O.Proj(p["suh"].numpy(), p["svh"].numpy(), trellis=p["trellis"].numpy(), K=K) for p in ex)
           for ex in experts]
    ref = O.moe_layer(x.numpy(), orc, rid, rw, O.ACT_SILU)
    assert np.abs(y.cpu().numpy() - ref).max() / np.abs(ref).max() <= 2e-3
    for b, h in zip(blobs, host):
        assert np.array_equal(b.cpu().numpy(), h)
    # the reference op returns x's dtype
    y16 = exl3.moe_forward_blobs(x.cuda(), ids, w, ptrs, I, K, E)
    assert y16.dtype == torch.float16 and np.abs(y16.float().cpu().numpy() - ref).max() / np.abs(ref).max() <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("K", [3, 6])
def test_blob_unplanarize_then_tile_order_reads_the_same_layer(exl3, K):
    """The optional conversion: blob_unplanarize puts each blob's words into tile order (equal to the oracle's tile-
    order words), and the tile-order read of the converted blobs gives the PLANAR4 read's layer bit for bit."""
    H, I, E = 256, 384, 6
    experts = [_expert(H, I, K, K, 1500 + 10 * e) for e in range(E)]
    host = [O.reference_blob(*[{k: v.numpy() for k, v in p.items()} for p in ex], K) for ex in experts]
    blobs = [torch.from_numpy(b).cuda() for b in host]
    ptrs = torch.tensor([b.data_ptr() for b in blobs], dtype=torch.int64, device="cuda")
    g = torch.Generator().manual_seed(1600 + K)
    x = torch.randn(5, H, generator=g).half().cuda()
    rid, rw = O.route_softmax_topk(torch.randn(5, E, generator=g).numpy(), 2)
    ids = torch.from_numpy(rid.astype(np.int32)).cuda()
    w = torch.from_numpy(rw.astype(np.float32)).cuda()
    y_pl = exl3.moe_forward_blobs(x, ids, w, ptrs, I, K, E, out_dtype=torch.float32)
    exl3.blob_unplanarize(ptrs, H, I, K)
    for ex, b in zip(experts, blobs):
        gu = np.concatenate([ex[0]["trellis"].numpy(), ex[1]["trellis"].numpy()], axis=1)
        nw = gu.size // 2
        words = b.cpu().numpy().view(np.uint32)
        assert np.array_equal(words[:nw], np.ascontiguousarray(gu).view(np.uint32).reshape(-1))
        assert np.array_equal(words[nw:nw + ex[2]["trellis"].numel() // 2],
                              np.ascontiguousarray(ex[2]["trellis"].numpy()).view(np.uint32).reshape(-1))
    y_t = exl3.moe_forward_blobs(x, ids, w, ptrs, I, K, E, out_dtype=torch.float32, tile_order=True)
    assert torch.equal(y_pl, y_t)


@pytest.mark.gpu
def test_moe_forward_blobs_bf16_x(exl3):
    """bf16 x, as the reference op accepts it: rows converted to fp16 before the input transform and the fp32 layer
    output rounded once to bf16 (the reference kernel's block-load conversion and its combine store), against the
    oracle's layer on the fp16-converted rows."""
    H, I, K, E = 256, 256, 3, 6
    experts = [_expert(H, I, K, K, 1700 + 10 * e) for e in range(E)]
    blobs = [torch.from_numpy(O.reference_blob(*[{k: v.numpy() for k, v in p.items()} for p in ex], K)).cuda()
             for ex in experts]
    ptrs = torch.tensor([b.data_ptr() for b in blobs], dtype=torch.int64, device="cuda")
    g = torch.Generator().manual_seed(1800)
    xb = torch.randn(4, H, generator=g).bfloat16()
    rid, rw = O.route_softmax_topk(torch.randn(4, E, generator=g).numpy(), 2)
    ids = torch.from_numpy(rid.astype(np.int32)).cuda()
    w = torch.from_numpy(rw.astype(np.float32)).cuda()
    y = exl3.moe_forward_blobs(xb.cuda(), ids, w, ptrs, I, K, E)
    assert y.dtype == torch.bfloat16
    orc = [tuple(O.Proj(p["suh"].numpy(), p["svh"].numpy(), trellis=p["trellis"].numpy(), K=K) for p in ex)
           for ex in experts]
    ref = O.moe_layer(xb.half().numpy(), orc, rid, rw, O.ACT_SILU)
    # 2e-3 for the layer plus half a bf16 ulp (2^-9 relative) for the final rounding
    assert np.abs(y.float().cpu().numpy() - ref).max() / np.abs(ref).max() <= 2e-3 + 2 ** -9
