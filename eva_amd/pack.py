"""DS41PK01 expert packs: read a pack's index, load whole layers into HBM, write packs.

A DS41PK01 pack is the reference's on-disk form of the routed EXL3 experts (writer
tools/pack_exl3.py:13-206; readers runtime/ds41/cache.py:40-43,150-158,1788-1797 and
tools/repack_expert_alignment.py:25-31). Every multi-byte field is little-endian:

- header, 24 bytes: ``b"DS41PK01"`` then uint32 version (1), n_layers, n_experts, slot bytes
  (128);
- index from byte 24: ``n_layers * n_experts`` records of ``slot`` bytes, layer-major, each
  ``<QIHH`` (record offset, record bytes padded to 4 KiB, K of w1, flag) followed by three
  projection blocks ``<HHHHIIIiIII`` in the order w1, w2, w3: in_features, out_features, K
  (trellis last dimension // 16), 0, suh bytes, svh bytes, trellis bytes, mul1 marker, and the
  suh / svh / trellis byte offsets inside the record;
- payload: the records, each a multiple of 4 KiB.

w1 is the gate projection, w3 the up projection and w2 the down projection (cache.py:1865-1886);
suh and svh are fp16 vectors, the trellis is int16 ``[in/16, out/16, 16*K]`` (``16*b+8`` at the
half rates b+0.5, which the K field cannot express: the rate is taken from the trellis size).

On a 288 GB MI355X every expert of the model fits in HBM, so there is no VRAM/RAM/NVMe tiering
here: ``load_layers`` streams each layer's contiguous byte range through a pinned host buffer
into one device allocation and builds the ``[9, n_experts]`` pointer table the kernels read.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np
import torch

MAGIC = b"DS41PK01"
HEADER = struct.Struct("<8sIIII")
SLOT_FMT = struct.Struct("<QIHH" + "HHHHIIIiIII" * 3)
SLOT_BYTES = 128
ALIGN = 4096
PROJ_ORDER = ("w1", "w2", "w3")          # gate, down, up, as stored
TABLE_PROJ = ("w1", "w3", "w2")          # pointer-table order: gate, up, down


@dataclass(frozen=True)
class ProjRecord:
    in_features: int
    out_features: int
    k: int
    suh_bytes: int
    svh_bytes: int
    trellis_bytes: int
    mul1: int
    rel_suh: int
    rel_svh: int
    rel_trellis: int

    @property
    def tile_u16(self) -> int:
        tiles = (self.in_features // 16) * (self.out_features // 16)
        return self.trellis_bytes // (2 * tiles)

    @property
    def bits(self) -> float:
        """Rate from the trellis size: 16*K uint16 per tile, or 16*b+8 at rate b+0.5."""
        t = self.tile_u16
        return t / 16 if t % 16 == 0 else (t - 8) / 16 + 0.5


@dataclass(frozen=True)
class ExpertRecord:
    offset: int
    nbytes: int
    k0: int
    flag: int
    projs: tuple            # ProjRecord for w1, w2, w3

    def proj(self, name: str) -> ProjRecord:
        return self.projs[PROJ_ORDER.index(name)]


@dataclass
class PackIndex:
    path: str
    version: int
    n_layers: int
    n_experts: int
    slot_bytes: int
    records: list           # [layer][expert] -> ExpertRecord

    def layer_span(self, layer: int):
        """Byte range [start, end) of a layer's records (they are stored contiguously)."""
        recs = self.records[layer]
        start = min(r.offset for r in recs)
        end = max(r.offset + r.nbytes for r in recs)
        return start, end


def parse_slot(raw: bytes) -> ExpertRecord:
    f = SLOT_FMT.unpack_from(raw)
    projs = []
    for pi in range(3):
        b = 4 + 11 * pi
        in_f, out_f, k, _pad, suh_b, svh_b, tr_b, mul1, r_suh, r_svh, r_tr = f[b:b + 11]
        projs.append(ProjRecord(in_f, out_f, k, suh_b, svh_b, tr_b, mul1, r_suh, r_svh, r_tr))
    return ExpertRecord(f[0], f[1], f[2], f[3], tuple(projs))


def read_index(path: str) -> PackIndex:
    """Parse a pack's header and index (no payload is read). Raises ValueError on a malformed pack."""
    size = os.path.getsize(path)
    with open(path, "rb") as fh:
        head = fh.read(HEADER.size)
        if len(head) != HEADER.size:
            raise ValueError(f"{path}: shorter than the 24-byte header")
        magic, version, n_layers, n_experts, slot = HEADER.unpack(head)
        if magic != MAGIC:
            raise ValueError(f"{path}: bad pack magic {magic!r}")
        if version != 1 or slot != SLOT_BYTES or n_layers < 1 or n_experts < 1:
            raise ValueError(f"{path}: unsupported pack (version {version}, slot {slot}, "
                             f"{n_layers} layers, {n_experts} experts)")
        raw = fh.read(n_layers * n_experts * slot)
    if len(raw) != n_layers * n_experts * slot:
        raise ValueError(f"{path}: index truncated")
    records = []
    for l in range(n_layers):
        row = []
        for e in range(n_experts):
            r = parse_slot(raw[(l * n_experts + e) * slot:(l * n_experts + e + 1) * slot])
            if r.offset < HEADER.size + len(raw) or r.offset + r.nbytes > size:
                raise ValueError(f"{path}: record ({l}, {e}) at {r.offset}+{r.nbytes} outside the payload")
            for p in r.projs:
                if p.in_features % 16 or p.out_features % 16 or p.suh_bytes != 2 * p.in_features \
                        or p.svh_bytes != 2 * p.out_features:
                    raise ValueError(f"{path}: record ({l}, {e}) has inconsistent projection sizes")
                for rel, n in ((p.rel_suh, p.suh_bytes), (p.rel_svh, p.svh_bytes), (p.rel_trellis, p.trellis_bytes)):
                    if rel % 2 or rel + n > r.nbytes:
                        raise ValueError(f"{path}: record ({l}, {e}) has a tensor outside the record")
            row.append(r)
        records.append(row)
    return PackIndex(path, version, n_layers, n_experts, slot, records)


class ResidentLayer:
    """One layer's experts in one device allocation, with its pointer table and rates."""

    def __init__(self, index: PackIndex, layer: int, storage: torch.Tensor, base: int):
        self.layer = layer
        self.storage = storage
        dev_base = storage.data_ptr()
        recs = index.records[layer]
        rows = [[0] * len(recs) for _ in range(9)]
        k2, k2d = [], []
        for e, r in enumerate(recs):
            for t, name in enumerate(TABLE_PROJ):
                p = r.proj(name)
                at = dev_base + (r.offset - base)
                rows[3 * t + 0][e] = at + p.rel_trellis
                rows[3 * t + 1][e] = at + p.rel_suh
                rows[3 * t + 2][e] = at + p.rel_svh
            # gate (w1) and up (w3) share one rate, as the reference's converter allocates them as
            # one group; down (w2) may differ (the coop launcher's K_gu / K_d)
            gu = {r.proj("w1").bits, r.proj("w3").bits}
            if len(gu) != 1:
                raise ValueError(f"layer {layer} expert {e}: gate and up at different rates {sorted(gu)}")
            k2.append(int(round(2 * gu.pop())))
            k2d.append(int(round(2 * r.proj("w2").bits)))
        self.table = torch.tensor(rows, dtype=torch.int64, device=storage.device)
        self.k2_host = tuple(k2)
        self.k2 = torch.tensor(k2, dtype=torch.uint8, device=storage.device)
        self.k2_down_host = tuple(k2d)
        self.k2_down = torch.tensor(k2d, dtype=torch.uint8, device=storage.device)
        r0 = recs[0]
        self.hidden = r0.proj("w1").in_features
        self.inter = r0.proj("w1").out_features


def load_layers(index: PackIndex, layers=None, device=None, chunk_bytes: int = 256 << 20) -> list:
    """Load layers' records into HBM: each layer's contiguous byte range is read through a pinned
    host buffer of ``chunk_bytes`` and copied to one device tensor. Returns ResidentLayer objects."""
    dev = torch.device("cuda", 0) if device is None else torch.device(device)
    layers = range(index.n_layers) if layers is None else layers
    pinned = torch.empty(chunk_bytes, dtype=torch.uint8, pin_memory=True)
    out = []
    fd = os.open(index.path, os.O_RDONLY)
    try:
        for l in layers:
            start, end = index.layer_span(l)
            storage = torch.empty(end - start, dtype=torch.uint8, device=dev)
            done = 0
            view = memoryview(pinned.numpy())
            while done < end - start:
                n = min(chunk_bytes, end - start - done)
                got = os.preadv(fd, [view[:n]], start + done)
                if got != n:
                    raise OSError(f"{index.path}: short read at {start + done}")
                storage[done:done + n].copy_(pinned[:n])       # synchronous: the buffer is reused next
                done += n
            out.append(ResidentLayer(index, l, storage, start))
    finally:
        os.close(fd)
    return out


def write_pack(path: str, layers, mul1: int = 1, align_first: bool = True) -> None:
    """Write a DS41PK01 pack. ``layers[l][e]`` maps ``"w1"``, ``"w2"``, ``"w3"`` to (suh fp16,
    svh fp16, trellis int16) numpy arrays. Records are padded to 4 KiB like the reference writer;
    with ``align_first`` the payload also starts on a 4 KiB boundary (the aligned layout of
    tools/repack_expert_alignment.py)."""
    n_layers = len(layers)
    n_experts = len(layers[0])
    index_bytes = n_layers * n_experts * SLOT_BYTES
    cursor = HEADER.size + index_bytes
    if align_first:
        cursor = (cursor + ALIGN - 1) & ~(ALIGN - 1)
    slots, blobs = [], []
    for l in range(n_layers):
        for e in range(n_experts):
            ex = layers[l][e]
            rel, fields, parts = 0, [], []
            for name in PROJ_ORDER:
                suh, svh, tr = (np.ascontiguousarray(a) for a in ex[name])
                if suh.dtype != np.float16 or svh.dtype != np.float16 or tr.dtype != np.int16:
                    raise ValueError("suh/svh must be float16 and the trellis int16")
                r_suh, r_svh, r_tr = rel, rel + suh.nbytes, rel + suh.nbytes + svh.nbytes
                rel = r_tr + tr.nbytes
                fields.extend([suh.shape[0], svh.shape[0], tr.shape[-1] // 16, 0, suh.nbytes, svh.nbytes, tr.nbytes,
                               mul1, r_suh, r_svh, r_tr])
                parts += [suh.tobytes(), svh.tobytes(), tr.tobytes()]
            padded = (rel + ALIGN - 1) & ~(ALIGN - 1)
            k0 = fields[2]
            slots.append(SLOT_FMT.pack(cursor, padded, k0, 1, *fields).ljust(SLOT_BYTES, b"\0"))
            blobs.append((cursor, b"".join(parts)))
            cursor += padded
    with open(path, "wb") as fh:
        fh.truncate(cursor)
        fh.write(HEADER.pack(MAGIC, 1, n_layers, n_experts, SLOT_BYTES))
        fh.write(b"".join(slots))
        for at, data in blobs:
            fh.seek(at)
            fh.write(data)
