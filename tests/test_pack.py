"""DS41PK01 expert packs on the host: the index format against a hand-built record, round trips
of written packs (fields, alignment, tensor bytes), rate inference and malformed packs
(format: tools/pack_exl3.py:13-206, runtime/ds41/cache.py:40-43,150-158,1788-1797)."""
import os
import struct

import numpy as np
import pytest

from eva_amd import pack
from oracle import exl3, synth


def _expert(rng, H, I, K):
    ew = synth.expert(rng, H, I, K)
    # oracle parts are (trellis, suh, svh) for g/u/d; a pack stores (suh, svh, trellis) for w1/w2/w3
    part = lambda p: (ew.parts[p][1], ew.parts[p][2], ew.parts[p][0])
    return {"w1": part("g"), "w2": part("d"), "w3": part("u")}, ew


def test_slot_layout_known_answer():
    # the reference's slot struct, field by field (tools/pack_exl3.py:73, cache.py:41)
    assert pack.SLOT_FMT.format == "<QIHH" + "HHHHIIIiIII" * 3
    assert pack.SLOT_FMT.size == 16 + 3 * 36 == 124
    fields = [123456789012, 8192, 4, 1]
    for pi in range(3):
        fields += [7168 if pi != 1 else 2048, 2048 if pi != 1 else 7168, 4, 0, 111 + pi, 222 + pi, 333 + pi,
                   -5 - pi, 10 * pi, 20 * pi, 30 * pi]
    raw = struct.pack("<QIHH" + "HHHHIIIiIII" * 3, *fields).ljust(128, b"\0")
    r = pack.parse_slot(raw)
    assert (r.offset, r.nbytes, r.k0, r.flag) == (123456789012, 8192, 4, 1)
    assert r.proj("w2") == pack.ProjRecord(2048, 7168, 4, 112, 223, 334, -6, 10, 20, 30)
    assert r.proj("w1").mul1 == -5 and r.proj("w3").rel_trellis == 60


@pytest.mark.parametrize("align_first", [False, True])
def test_write_read_round_trip(tmp_path, align_first):
    rng = np.random.default_rng(7)
    H, I = 256, 128
    rates = [[2, 2.5, 4], [3, 5, 1.5]]
    layers, src = [], []
    for row in rates:
        exps = [_expert(rng, H, I, K) for K in row]
        layers.append([e for e, _ in exps])
        src.append([e for e, _ in exps])
    path = str(tmp_path / "experts.bin")
    pack.write_pack(path, layers, mul1=0x1234, align_first=align_first)
    idx = pack.read_index(path)
    assert (idx.version, idx.n_layers, idx.n_experts, idx.slot_bytes) == (1, 2, 3, 128)
    raw = open(path, "rb").read()
    end_of_index = 24 + 2 * 3 * 128
    prev = None
    for l, row in enumerate(rates):
        for e, K in enumerate(row):
            r = idx.records[l][e]
            assert r.nbytes % 4096 == 0 and r.flag == 1
            assert r.offset >= end_of_index
            if align_first:
                assert r.offset % 4096 == 0
            if prev is not None:
                assert r.offset == prev.offset + prev.nbytes           # layer-major, contiguous
            prev = r
            for name in pack.PROJ_ORDER:
                p = r.proj(name)
                suh, svh, tr = src[l][e][name]
                assert p.bits == K and p.tile_u16 == exl3.tile_u16(K) and p.mul1 == 0x1234
                assert p.k == tr.shape[-1] // 16
                got = lambda rel, n, dt: np.frombuffer(raw[r.offset + rel:r.offset + rel + n], dtype=dt)
                assert np.array_equal(got(p.rel_suh, p.suh_bytes, np.float16).view(np.uint16), suh.view(np.uint16))
                assert np.array_equal(got(p.rel_svh, p.svh_bytes, np.float16).view(np.uint16), svh.view(np.uint16))
                assert np.array_equal(got(p.rel_trellis, p.trellis_bytes, np.int16), tr.reshape(-1))
        start, end = idx.layer_span(l)
        assert end - start == sum(r.nbytes for r in idx.records[l])


def test_malformed_packs_are_rejected(tmp_path):
    rng = np.random.default_rng(8)
    e, _ = _expert(rng, 128, 128, 2)
    path = str(tmp_path / "p.bin")
    pack.write_pack(path, [[e]])
    good = open(path, "rb").read()
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"DS41PK02" + good[8:])
    with pytest.raises(ValueError, match="magic"):
        pack.read_index(str(bad))
    bad.write_bytes(good[:24 + 64])
    with pytest.raises(ValueError, match="truncated"):
        pack.read_index(str(bad))
    # a record that points past the end of the file
    rec = bytearray(good[24:24 + 128])
    struct.pack_into("<Q", rec, 0, len(good))
    bad.write_bytes(good[:24] + bytes(rec) + good[24 + 128:])
    with pytest.raises(ValueError, match="outside"):
        pack.read_index(str(bad))
    bad.write_bytes(good[:8] + struct.pack("<IIII", 2, 1, 1, 128) + good[24:])
    with pytest.raises(ValueError, match="unsupported"):
        pack.read_index(str(bad))
