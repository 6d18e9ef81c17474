"""Expert records: one contiguous arena per routed expert, experts of a layer at a uniform stride in one device
allocation, and a layer-major record store on disk.

Record layout (format "exl3mi-expert-v1"; every section 256-byte aligned, the record padded to 4096 bytes):
    gate.trellis int16 [H/16, I/16, 16 Kgu] | up.trellis | down.trellis int16 [I/16, H/16, 16 Kd] |
    gate.suh fp16 [H] | gate.svh [I] | up.suh [H] | up.svh [I] | down.suh [I] | down.svh [H]
This is the section order of the reference's NVMe expert record (glm/xpu/pack_store.py:14-19) with the trellis words in
their checkpoint (standard tile) order, which is what the MI355X kernels read: a record is one contiguous copy from disk
to HBM, and an arena of records gives ExpertTables rows base + e * stride, the layout the decode kernels address
without loading tables.

The reference's own expert blob (pack_expert, glm/xpu/exl3xpu/moe_offload.py:81-94; byte offsets in Geom,
glm/xpu/csrc/exl3_moe.n128.sycl:56-68) keeps gate|up (concatenated along the columns) and down in PLANAR4 word order
(planar4, moe_offload.py:68-78; blob_perm, pack_store.py:35-60) followed by g.suh u.suh g.svh u.svh d.suh d.svh.
unpack_reference_blob inverts that permutation, so experts packed for the reference load here by a repack only.
"""
from __future__ import annotations

import hashlib
import json
import math
import os

import numpy as np
import torch

from ._lib import Exl3Error
from .linear import BC_LinearEXL3

FORMAT = "exl3mi-expert-v1"
SECTION_ALIGN = 256
RECORD_ALIGN = 4096


def _up(n: int, a: int) -> int:
    return (n + a - 1) // a * a


class RecordGeom:
    """Byte layout of one expert record for hidden size H, intermediate size I, gate/up bits Kgu and down bits Kd."""

    def __init__(self, H: int, I: int, Kgu: int, Kd: int | None = None):
        Kd = Kgu if Kd is None else Kd
        if H % 128 or I % 128 or not (1 <= Kgu <= 8) or not (1 <= Kd <= 8):
            raise Exl3Error(f"RecordGeom: H={H}, I={I} must be multiples of 128 and K in 1..8 (got {Kgu}, {Kd})")
        self.H, self.I, self.Kgu, self.Kd = H, I, Kgu, Kd
        shapes = [("gate.trellis", (H // 16, I // 16, 16 * Kgu), torch.int16),
                  ("up.trellis", (H // 16, I // 16, 16 * Kgu), torch.int16),
                  ("down.trellis", (I // 16, H // 16, 16 * Kd), torch.int16),
                  ("gate.suh", (H,), torch.float16), ("gate.svh", (I,), torch.float16),
                  ("up.suh", (H,), torch.float16), ("up.svh", (I,), torch.float16),
                  ("down.suh", (I,), torch.float16), ("down.svh", (H,), torch.float16)]
        self.sections = {}
        off = 0
        for name, shape, dt in shapes:
            nb = math.prod(shape) * 2
            self.sections[name] = (off, nb, shape, dt)
            off = _up(off + nb, SECTION_ALIGN)
        self.bytes = _up(off, RECORD_ALIGN)

    def to_json(self) -> dict:
        return {"H": self.H, "I": self.I, "Kgu": self.Kgu, "Kd": self.Kd, "record_bytes": self.bytes}


def _fields(p) -> dict:
    if isinstance(p, dict):
        return p
    return {"trellis": p.trellis, "suh": p.suh, "svh": p.svh}


def pack_expert(gate, up, down, geom: RecordGeom, out: torch.Tensor | None = None) -> torch.Tensor:
    """One expert (gate, up, down as BC_LinearEXL3 or {trellis, suh, svh} dicts) -> record bytes (uint8 [geom.bytes],
    on `out`'s device when given, else on the CPU)."""
    if out is None:
        out = torch.zeros(geom.bytes, dtype=torch.uint8)
    if out.dtype != torch.uint8 or out.numel() != geom.bytes or not out.is_contiguous():
        raise Exl3Error(f"pack_expert: out must be contiguous uint8 [{geom.bytes}]")
    for proj, p in (("gate", gate), ("up", up), ("down", down)):
        f = _fields(p)
        for kind in ("trellis", "suh", "svh"):
            off, nb, shape, dt = geom.sections[f"{proj}.{kind}"]
            t = f[kind]
            if tuple(t.shape) != shape or t.dtype != dt:
                raise Exl3Error(f"pack_expert: {proj}.{kind} must be {dt} {shape}, got {t.dtype} {tuple(t.shape)}")
            out[off:off + nb].copy_(t.contiguous().view(-1).view(torch.uint8))
    return out


def expert_views(rec: torch.Tensor, geom: RecordGeom):
    """(gate, up, down) BC_LinearEXL3 whose tensors are views into one record's bytes (no copy)."""
    v = {}
    for name, (off, nb, shape, dt) in geom.sections.items():
        v[name] = rec[off:off + nb].view(dt).view(shape)
    return tuple(BC_LinearEXL3(v[f"{p}.trellis"], v[f"{p}.suh"], v[f"{p}.svh"], geom.Kgu if p != "down" else geom.Kd,
                               None, False, True, None) for p in ("gate", "up", "down"))


class ExpertArena:
    """E expert records in one allocation (record e at byte e * geom.bytes)."""

    def __init__(self, E: int, geom: RecordGeom, device="cuda", buf: torch.Tensor | None = None):
        self.E, self.geom = E, geom
        if buf is None:
            buf = torch.zeros(E * geom.bytes, dtype=torch.uint8, device=device)
        if buf.dtype != torch.uint8 or buf.numel() != E * geom.bytes or not buf.is_contiguous():
            raise Exl3Error(f"ExpertArena: buffer must be contiguous uint8 [{E * geom.bytes}]")
        self.buf = buf

    def record(self, e: int) -> torch.Tensor:
        return self.buf[e * self.geom.bytes:(e + 1) * self.geom.bytes]

    def put(self, e: int, gate, up, down) -> None:
        pack_expert(gate, up, down, self.geom, self.record(e))

    def experts(self):
        return [expert_views(self.record(e), self.geom) for e in range(self.E)]

    def tables(self, extra=None):
        """ExpertTables over the arena (uniform strides). `extra`: an optional (gate, up, down) appended as the last
        entry (a shared expert; the table rows then stay uniform only if it lives in the arena's stride pattern)."""
        from .moe import ExpertTables
        ex = self.experts()
        if extra is not None:
            ex.append(tuple(extra))
        return ExpertTables([g for g, _, _ in ex], [u for _, u, _ in ex], [d for _, _, d in ex])


# ------------------------------------------------------------------------------------------------ reference blob
def _planar4_dims(K: int):
    D = K // math.gcd(K, 32)          # words per period
    return D, 8 * K // D              # (D, G periods per tile)


def unplanar4(words: torch.Tensor, rows: int, tiles: int, K: int) -> torch.Tensor:
    """Inverse of the reference's PLANAR4 word order: words [rows][tiles / 4][D][4][G] -> int32 [rows, tiles, 8K] in
    tile order (identity when D = 1, i.e. K = 2, 4, 8)."""
    D, G = _planar4_dims(K)
    if tiles % 4:
        raise Exl3Error("unplanar4: tiles per row must be a multiple of 4")
    w = words.reshape(rows, tiles // 4, D, 4, G)
    return w.permute(0, 1, 3, 4, 2).reshape(rows, tiles, 8 * K).contiguous()


def unpack_reference_blob(blob: torch.Tensor, H: int, I: int, K: int):
    """The reference's exl3xpu expert blob (uint8, pack_expert layout) -> (gate, up, down) dicts of int16 trellis and
    fp16 suh / svh in checkpoint order (CPU tensors)."""
    b = blob.contiguous().view(torch.uint8).cpu()
    W = 8 * K
    gu_words = (H // 16) * (2 * I // 16) * W
    d_words = (I // 16) * (H // 16) * W
    need = 4 * (gu_words + d_words) + 2 * (3 * H + 3 * I)
    if b.numel() < need:
        raise Exl3Error(f"unpack_reference_blob: blob of {b.numel()} bytes, need {need}")
    w = b[:4 * (gu_words + d_words)].view(torch.int32)
    gu = unplanar4(w[:gu_words], H // 16, 2 * I // 16, K).view(torch.int16).view(H // 16, 2 * I // 16, 16 * K)
    dn = unplanar4(w[gu_words:], I // 16, H // 16, K).view(torch.int16).view(I // 16, H // 16, 16 * K)
    o = 4 * (gu_words + d_words)
    vec = {}
    for name, n in (("g_suh", H), ("u_suh", H), ("g_svh", I), ("u_svh", I), ("d_suh", I), ("d_svh", H)):
        vec[name] = b[o:o + 2 * n].view(torch.float16).clone()
        o += 2 * n
    gate = {"trellis": gu[:, :I // 16].contiguous(), "suh": vec["g_suh"], "svh": vec["g_svh"]}
    up = {"trellis": gu[:, I // 16:].contiguous(), "suh": vec["u_suh"], "svh": vec["u_svh"]}
    down = {"trellis": dn, "suh": vec["d_suh"], "svh": vec["d_svh"]}
    return gate, up, down


# ------------------------------------------------------------------------------------------------ store
def write_store(path: str, layers) -> dict:
    """Write a layer-major record store: `path`.bin holds every layer's records (layer li at its own offset, record
    e at offset + e * record_bytes), `path`.json the layout and the sha256 of every record. `layers` is a sequence of
    (RecordGeom, experts) with experts a sequence of (gate, up, down). Returns the manifest."""
    man = {"format": FORMAT, "layers": []}
    off = 0
    with open(path + ".bin", "wb") as f:
        for geom, experts in layers:
            hashes = []
            for gate, up, down in experts:
                rec = pack_expert(gate, up, down, geom)
                raw = rec.numpy().tobytes()
                hashes.append(hashlib.sha256(raw).hexdigest())
                f.write(raw)
            man["layers"].append({**geom.to_json(), "E": len(hashes), "offset": off, "sha256": hashes})
            off += len(hashes) * geom.bytes
    with open(path + ".json", "w") as f:
        json.dump(man, f)
    return man


def read_manifest(path: str) -> dict:
    with open(path + ".json") as f:
        man = json.load(f)
    if man.get("format") != FORMAT:
        raise Exl3Error(f"{path}.json: format {man.get('format')!r}, expected {FORMAT!r}")
    return man


def _layer_bytes(path: str, lay: dict) -> np.ndarray:
    n = lay["E"] * lay["record_bytes"]
    with open(path + ".bin", "rb") as f:
        f.seek(lay["offset"])
        raw = np.frombuffer(f.read(n), dtype=np.uint8)
    if raw.size != n:
        raise Exl3Error(f"{path}.bin: short read of layer at {lay['offset']}")
    return raw


def verify_store(path: str) -> list:
    """(layer, expert) of every record whose bytes do not match the manifest's sha256."""
    man = read_manifest(path)
    bad = []
    for li, lay in enumerate(man["layers"]):
        raw = _layer_bytes(path, lay)
        rb = lay["record_bytes"]
        for e, h in enumerate(lay["sha256"]):
            if hashlib.sha256(raw[e * rb:(e + 1) * rb].tobytes()).hexdigest() != h:
                bad.append((li, e))
    return bad


def load_layer(path: str, li: int, device="cuda", verify: bool = True) -> ExpertArena:
    """Layer li of a store as an ExpertArena on `device` (one host read, one copy to the device)."""
    man = read_manifest(path)
    lay = man["layers"][li]
    geom = RecordGeom(lay["H"], lay["I"], lay["Kgu"], lay["Kd"])
    if geom.bytes != lay["record_bytes"]:
        raise Exl3Error(f"{path}: record size {lay['record_bytes']} does not match the layout ({geom.bytes})")
    raw = _layer_bytes(path, lay)
    if verify:
        rb = geom.bytes
        for e, h in enumerate(lay["sha256"]):
            if hashlib.sha256(raw[e * rb:(e + 1) * rb].tobytes()).hexdigest() != h:
                raise Exl3Error(f"{path}: layer {li} expert {e} fails its sha256")
    buf = torch.from_numpy(raw.copy()).to(device)
    return ExpertArena(lay["E"], geom, device, buf)
