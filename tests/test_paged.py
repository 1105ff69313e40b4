"""Paged expert-pool feed: the .vq2m container reader / writer and the LRU
pager run on the CPU here; the GPU parity of PagedMoEExperts against the
resident pool is in test_gpu_parity.py."""
import os
import struct

import numpy as np
import pytest
import torch

from compressai_amd import paged


def _layers(L, E, gu=(32, 16), dn=(64, 4), seed=0):
    g = torch.Generator().manual_seed(seed)
    gui = [torch.randint(-32768, 32768, (E, *gu), generator=g, dtype=torch.int32).to(torch.int16) for _ in range(L)]
    gus = [(torch.rand(E, gu[0], generator=g) + 0.5).to(torch.float16) for _ in range(L)]
    dni = [torch.randint(-32768, 32768, (E, *dn), generator=g, dtype=torch.int32).to(torch.int16) for _ in range(L)]
    dns = [(torch.rand(E, dn[0], generator=g) + 0.5).to(torch.float16) for _ in range(L)]
    return gui, gus, dni, dns


def _record(t, l, e):
    return b"".join(x[l][e].contiguous().view(torch.uint8).numpy().tobytes() for x in t)


def test_container_round_trip(tmp_path):
    t = _layers(2, 5)
    path = tmp_path / "m.vq2m"
    paged.write_vq2m(path, *t, meta={"expert_modes": {"1:3": 3}})
    st = paged.Vq2mStore(path)
    assert (st.num_layers, st.num_experts) == (2, 5)
    assert (st.gu_rows, st.gu_cols, st.dn_rows, st.dn_cols) == (32, 16, 64, 4)
    assert st.record_bytes == 32 * 16 * 2 + 32 * 2 + 64 * 4 * 2 + 64 * 2
    assert st.promoted(1, 3) and not st.promoted(0, 3)
    # header fields at the reference's byte positions
    head = open(path, "rb").read(64)
    assert head[:4] == b"VQ2M" and struct.unpack("<H", head[4:6])[0] == 1
    buf = bytearray(st.record_bytes)
    for l in range(2):
        for e in range(5):
            st.read_record(l, e, memoryview(buf))
            assert bytes(buf) == _record(t, l, e)
    st.close()


def test_non_contiguous_record_and_bad_files(tmp_path):
    t = _layers(1, 3, seed=1)
    path = tmp_path / "m.vq2m"
    paged.write_vq2m(path, *t)
    st = paged.Vq2mStore(path)
    # move expert 2's scale plane to the end of the file and point the table at it
    e = list(st.entries[0][2])
    data = open(path, "rb").read()
    moved = data[e[2]:e[2] + e[3]]
    with open(path, "ab") as f:
        new_off = f.tell()
        f.write(moved)
    with open(path, "r+b") as f:
        tbl_off = struct.unpack(paged.HEADER_FORMAT, data[:64])[5]
        e[2] = new_off
        f.seek(tbl_off + 2 * paged.ENTRY_SIZE)
        f.write(struct.pack(paged.ENTRY_FORMAT, *e))
    st2 = paged.Vq2mStore(path)
    buf = bytearray(st2.record_bytes)
    st2.read_record(0, 2, memoryview(buf))
    assert bytes(buf) == _record(t, 0, 2)
    st.close()
    st2.close()
    # a record whose sizes are not a 2 bpw expert (e.g. a promoted 3-bit one) is refused
    with open(path, "r+b") as f:
        e[1] += 2
        f.seek(tbl_off + 2 * paged.ENTRY_SIZE)
        f.write(struct.pack(paged.ENTRY_FORMAT, *e))
    with pytest.raises(ValueError):
        paged.Vq2mStore(path).read_record(0, 2, memoryview(buf))
    bad = tmp_path / "bad.vq2m"
    bad.write_bytes(b"NOPE" + bytes(60))
    with pytest.raises(ValueError):
        paged.Vq2mStore(bad)


def test_pager_lru_on_cpu(tmp_path):
    t = _layers(1, 8, seed=2)
    path = tmp_path / "m.vq2m"
    paged.write_vq2m(path, *t)
    st = paged.Vq2mStore(path)
    pg = paged.ExpertPager(st, 0, capacity=3, device="cpu", staging=2)
    s = pg.ensure([5, 1, 5])
    assert s[0] == s[2] and s[0] != s[1] and (pg.hits, pg.misses) == (1, 2)
    pg.ensure([2])                # pool now holds 5, 1, 2 (5 most recent of the first step)
    s2 = pg.ensure([1, 7])        # 7 evicts the least recently used: 5
    assert 5 not in pg.slot_of and set(pg.slot_of) == {2, 1, 7}
    assert s2[1] == s[0]          # 7 took 5's slot
    for e, slot in pg.slot_of.items():
        # the pool rounds the container's fp16 scales to bf16, as the reference's pools
        bf = torch.bfloat16
        assert torch.equal(pg.pool_gu_idx[slot], t[0][0][e]) and torch.equal(pg.pool_gu_scale[slot], t[1][0][e].to(bf))
        assert torch.equal(pg.pool_dn_idx[slot], t[2][0][e]) and torch.equal(pg.pool_dn_scale[slot], t[3][0][e].to(bf))
    with pytest.raises(RuntimeError):
        pg.ensure([0, 3, 4, 6])   # four distinct experts, three slots
    with pytest.raises(Exception):
        pg.ensure([8])            # outside the layer's experts
    st.close()


def test_promoted_records_round_trip(tmp_path):
    """Promoted (16,8) experts: the index entries hold the int16 plane then the
    uint8 plane (1.5x the 2 bpw entry), meta flags them, read_promoted returns
    the planes, and read_record refuses them."""
    t = _layers(2, 4, seed=5)
    g = torch.Generator().manual_seed(6)
    s2 = {(1, 2): (torch.randint(0, 256, (32, 16), generator=g, dtype=torch.int32).to(torch.uint8),
                   torch.randint(0, 256, (64, 4), generator=g, dtype=torch.int32).to(torch.uint8))}
    path = tmp_path / "p.vq2m"
    paged.write_vq2m(path, *t, promoted=s2)
    st = paged.Vq2mStore(path)
    assert st.promoted_experts(1) == [2] and st.promoted_experts(0) == []
    assert st.promoted_sizes == (32 * 16 * 3, 32 * 2, 64 * 4 * 3, 64 * 2)
    r = st.read_promoted(1, 2)
    gui, gus, dni, dns = t
    assert torch.equal(r["gu0"], gui[1][2]) and torch.equal(r["gu1"], s2[(1, 2)][0])
    assert torch.equal(r["dn0"], dni[1][2]) and torch.equal(r["dn1"], s2[(1, 2)][1])
    assert torch.equal(r["gu_s"], gus[1][2]) and torch.equal(r["dn_s"], dns[1][2])
    # the gate_up index entry is the two planes back to back
    off, sz = st.entries[1][2][0], st.entries[1][2][1]
    raw = open(path, "rb").read()[off:off + sz]
    assert raw == gui[1][2].numpy().tobytes() + s2[(1, 2)][0].numpy().tobytes()
    with pytest.raises(ValueError, match="promoted"):
        st.read_record(1, 2, memoryview(bytearray(st.record_bytes)))
    with pytest.raises(ValueError, match="not a promoted"):
        st.read_promoted(0, 2)
    # a regular record of the same layer still reads through the pager path
    buf = bytearray(st.record_bytes)
    st.read_record(1, 1, memoryview(buf))
    assert bytes(buf) == _record(t, 1, 1)
    st.close()


def test_promoted_layer_needs_stage2_codebook(tmp_path):
    t = _layers(1, 3, gu=(64, 16), dn=(128, 4), seed=7)
    s2 = {(0, 1): (torch.zeros(64, 16, dtype=torch.uint8), torch.zeros(128, 4, dtype=torch.uint8))}
    path = tmp_path / "q.vq2m"
    paged.write_vq2m(path, *t, promoted=s2)
    st = paged.Vq2mStore(path)
    cb = torch.zeros(65536, 8, dtype=torch.float16)
    with pytest.raises(Exception, match="cb8"):
        paged.PagedMoEExperts(0, st, cb, capacity=2, device="cpu")
    st.close()
