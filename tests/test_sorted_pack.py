"""The code-sorted repack (vq2_sorted_pack, host code of libvq2_amd.so) on the
CPU: every code of the planes appears exactly once in its chunk, with its row
and group; no row repeats inside a 32-lane half of an instruction (each
half read-add-writes its own accumulator array, so the kernel relies on
it); padding is the dummy row; and the instructions are sorted enough that
a wave's 64 gathers touch few codebook lines."""
import ctypes

import numpy as np
import pytest
import torch

from compressai_amd import _lib, synth
from compressai_amd.kernels import SortedPlanes, Vq2Error

def _gb(ng):
    return int(np.ceil(np.log2(ng))) if ng > 1 else 0


def _is_pad(v, sp):
    gb = _gb(sp.n // 8)
    return (v & 0xFFFF) == (sp.rows_per_chunk << gb)


def _decode(sp: SortedPlanes):
    """Per chunk and stage: list of instructions, each a (64,) uint32 array."""
    ent = sp.entries.cpu().numpy().view(np.uint32).reshape(-1, 64, 4)  # [iter][lane][q]
    ipc, ipc1 = sp.iters_per_chunk, sp.stage1_iters
    out = []
    for c in range(sp.n_chunks):
        stages = []
        for a, b in ((c * ipc, c * ipc + ipc1), (c * ipc + ipc1, (c + 1) * ipc)):
            stages.append([ent[it][:, q] for it in range(a, b) for q in range(4)])
        out.append(stages)
    return out


@pytest.mark.parametrize("rows,n,bpw", [(300, 2048, 2), (256, 2048, 4), (100, 6144, 4), (1000, 512, 2),
                                        (97, 800, 2), (5, 64, 4)])
def test_sorted_pack_is_a_permutation_with_distinct_rows(rows, n, bpw):
    ng = n // 8
    m = synth.vq_matrix(9800 + rows + bpw, rows, n, bpw=bpw)
    sp = SortedPlanes(m["idx0"], m["idx1"], rows, n, device="cpu", threads=3)
    R = int(_lib.load().vq2_sorted_rows_per_chunk(rows, ng, 1))
    gb = _gb(ng)
    assert sp.rows_per_chunk == R and (R + 1) * (1 << gb) <= 1 << 16
    assert sp.n_chunks == -(-rows // R) and R <= 255
    assert R * sp.n_chunks - rows < sp.n_chunks      # the rows split evenly over the chunks
    assert rows // sp.n_chunks + (1 if rows % sp.n_chunks else 0) <= R
    assert sp.n_iters == sp.n_chunks * sp.iters_per_chunk                 # chunks padded to one size
    assert 0 < sp.stage1_iters <= sp.iters_per_chunk
    assert (sp.stage1_iters < sp.iters_per_chunk) == (bpw == 4)
    planes = [m["idx0"].numpy().view(np.uint16)] + ([m["idx1"].numpy().view(np.uint16)] if bpw == 4 else [])
    for c, stages in enumerate(_decode(sp)):
        rb, nbig = rows // sp.n_chunks, rows % sp.n_chunks    # near-equal chunks: heights rb + 1 then rb
        r0 = c * rb + min(c, nbig)
        r1 = r0 + rb + (1 if c < nbig else 0)
        for st, instrs in enumerate(stages):
            if st >= len(planes):
                assert not instrs
                continue
            allv = np.concatenate(instrs) if instrs else np.zeros(0, np.uint32)
            real = allv[~_is_pad(allv, sp)]
            pad = allv[_is_pad(allv, sp)]
            assert np.all(pad >> 16 == 0)  # padding gathers code 0
            code, pos = real >> 16, real & 0xFFFF
            r, g = pos >> gb, pos & ((1 << gb) - 1)
            assert np.all(r < r1 - r0) and np.all(g < ng)
            got = np.zeros((r1 - r0, ng), np.int64) - 1
            assert len(real) == (r1 - r0) * ng          # every code exactly once ...
            got[r, g] = code
            assert np.array_equal(got, planes[st][r0:r1].astype(np.int64))  # ... at its row and group
            for ins in instrs:
                for qd in range(2):                      # no row twice in a 32-lane half
                    qv = ins[32 * qd:32 * qd + 32]
                    rr = (qv[~_is_pad(qv, sp)] & 0xFFFF) >> gb
                    assert len(np.unique(rr)) == len(rr)
            assert len(instrs) % 4 == 0


def test_sorted_pack_keeps_instructions_within_few_lines():
    """At the gate/up shape (6144 x 2048, 4 bpw) a 64-entry instruction of a
    255-row chunk (65280 codes) spans ~8-10 128-byte codebook lines (8 fp16
    centroids per line) instead of the ~64 of unsorted codes."""
    rows, n = 6144, 2048
    m = synth.vq_matrix(9900, rows, n, bpw=4)
    sp = SortedPlanes(m["idx0"], m["idx1"], rows, n, device="cpu")
    lines = []
    for stages in _decode(sp)[:8]:
        for instrs in stages:
            for ins in instrs:
                real = ins[~_is_pad(ins, sp)]
                if len(real) == 64:
                    lines.append(len(np.unique((real >> 16) >> 3)))
    assert 6 <= np.mean(lines) <= 12, np.mean(lines)
    print("mean codebook lines per instruction:", np.mean(lines))
    assert sp.n_iters <= 1.02 * (rows * n // 8 * 2) / 256  # little padding


def test_sorted_pack_rejects_bad_input():
    m = synth.vq_matrix(9910, 16, 512, bpw=3)
    with pytest.raises(Vq2Error):
        SortedPlanes(m["idx0"], m["idx1"], 16, 512, device="cpu")  # (16,8) is not covered
    with pytest.raises(Vq2Error):
        SortedPlanes(m["idx0"], None, 17, 512, device="cpu")      # wrong row count
    L = _lib.load()
    n_it, ipc, ipc1 = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
    buf = torch.empty(256, dtype=torch.int32)
    st = L.vq2_sorted_pack(m["idx0"].data_ptr(), None, 16, 64, 16, buf.data_ptr(), 1, ctypes.byref(ipc),
                           ctypes.byref(ipc1), ctypes.byref(n_it), 1)
    assert st == _lib.ERR_ARG and n_it.value > 1   # capacity too small: the needed size is reported
    assert n_it.value == ipc.value and ipc1.value == ipc.value
    st = L.vq2_sorted_pack(m["idx0"].data_ptr(), None, 16, 64, 256, buf.data_ptr(), 1000, ctypes.byref(ipc),
                           ctypes.byref(ipc1), ctypes.byref(n_it), 1)
    assert st == _lib.ERR_ARG                     # rows_per_chunk beyond the 16-bit position field


def test_sorted_rows_per_chunk_alignment():
    L = _lib.load()
    assert L.vq2_sorted_rows_per_chunk(151936, 256, 256) == 198   # 768 chunks: 3 rounds of 256 CUs
    assert L.vq2_sorted_rows_per_chunk(151936, 256, 1) == 255     # 596 chunks
    assert L.vq2_sorted_rows_per_chunk(6144, 256, 256) == 246     # 25 chunks (aligned ones would be too short)
    assert L.vq2_sorted_rows_per_chunk(2048, 768, 1) == 63        # 6144-wide: 63 rows at most (33 chunks)
    assert L.vq2_sorted_rows_per_chunk(100, 1 << 16, 1) == 0      # n beyond the 16-bit position field


@pytest.mark.parametrize("E,rows,n", [(3, 1024, 2048), (5, 2048, 512), (2, 100, 800)])
def test_sorted_pool_pack_equals_per_expert_pack(E, rows, n):
    """vq2_sorted_pack_pool lays the experts out one after another, each
    chunk exactly as vq2_sorted_pack packs it alone, then padded with
    dummy-row entries (code 0) to the pool's common iteration count."""
    from compressai_amd.kernels import SortedPool

    ng = n // 8
    idx = synth.indices16(9950 + rows, (E, rows, ng))
    pool = SortedPool(idx, device="cpu", threads=3)
    C, R = pool.chunks, pool.rows_per_chunk
    assert R == int(_lib.load().vq2_sorted_rows_per_chunk(rows, ng, 1)) and C == -(-rows // R)
    ipc = pool.iters_per_chunk
    assert pool.n_iters == E * C * ipc
    ent = pool.entries.numpy().view(np.uint32)
    pad = np.uint32(R << _gb(ng))
    longest = 0
    for e in range(E):
        sp = SortedPlanes(idx[e], None, rows, n, device="cpu", chunk_align=1)
        assert sp.rows_per_chunk == R and sp.n_chunks == C
        ipe = sp.iters_per_chunk   # this expert's chunks, padded to its own longest
        own = sp.entries.numpy().view(np.uint32)
        longest = max(longest, ipe)
        for c in range(C):
            got = ent[(e * C + c) * ipc * 256:(e * C + c + 1) * ipc * 256]
            assert np.array_equal(got[: ipe * 256], own[c * ipe * 256:(c + 1) * ipe * 256])
            assert np.all(got[ipe * 256:] == pad)
    assert ipc == longest


def test_moe_slices_cost_model():
    """Slice counts of the sorted MoE launches on 256 CUs: T = 1 fills one
    round (gate_up 45 units x 5, down 81 x 3); T = 8 takes 2 and 1."""
    from compressai_amd.kernels import moe_slices

    assert moe_slices(45, 205 * 256, 256, 2.5) == 5
    assert moe_slices(81, 228 * 64, 256, 2.0) == 3
    assert moe_slices(360, 205 * 256, 256, 2.5) == 2
    assert moe_slices(648, 228 * 64, 256, 2.0) == 1
