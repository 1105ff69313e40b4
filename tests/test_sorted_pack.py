"""The code-sorted repack (vq2_sorted_pack, host code of libvq2_amd.so) on the
CPU: every code of the planes appears exactly once in its chunk, with its row
and group; no row repeats inside a 32-lane half of an instruction, or a
16-lane quarter for chunks of at most 32 rows (each lane group
read-add-writes its own accumulator array, so the kernel relies on it);
lane 63 carries the instruction's smallest code and every offset fits
its field; padding is the dummy row at offset 0; and the instructions are
sorted enough that a wave's 64 gathers touch few codebook lines.

Format (3 bytes per code): an iteration is 64 lanes x 3 uint32; lane l
holds four 24-bit fields F_q = lo16_q | hi8_q << 16 (q = the iteration's
instruction), words lo16_0 | lo16_1 << 16, lo16_2 | lo16_3 << 16 and
hi8_0 | hi8_1 << 8 | hi8_2 << 16 | hi8_3 << 24.  Lane 63's lo16_q is the
base code of instruction q; every other field is
(code - base) << P | row << gbits | group, P = gbits + bitlen(R)."""
import ctypes

import numpy as np
import pytest
import torch

from compressai_amd import _lib, synth
from compressai_amd.kernels import ITER_WORDS, SortedPlanes, Vq2Error


def _gb(ng):
    return int(np.ceil(np.log2(ng))) if ng > 1 else 0


def _pb(ng, R):
    return _gb(ng) + int(R).bit_length()


def _fields(words):
    """uint32 [iters * 192] -> (F [iters, 64, 4] 24-bit fields, lo16, hi8)."""
    w = words.reshape(-1, 64, 3).astype(np.uint32)
    lo = np.stack([w[..., 0] & 0xFFFF, w[..., 0] >> 16, w[..., 1] & 0xFFFF, w[..., 1] >> 16], axis=-1)
    hi = np.stack([(w[..., 2] >> (8 * q)) & 0xFF for q in range(4)], axis=-1)
    return lo | (hi << 16), lo, hi


def _decode_words(words, ng, R):
    """Per instruction (iteration-major, then q): (codes [63], positions [63],
    base, offsets [63])."""
    F, lo, hi = _fields(words)
    pb = _pb(ng, R)
    assert np.all(hi[:, 63, :] == 0)  # the base lane's high bytes are zero
    out = []
    for it in range(F.shape[0]):
        for q in range(4):
            f = F[it, :63, q]
            base = int(lo[it, 63, q])
            off = f >> pb
            assert np.all(off < (1 << (24 - pb)))
            out.append(((base + off) & 0xFFFF, f & ((1 << pb) - 1), base, off))
    return out


def _decode(sp: SortedPlanes):
    """Per chunk and stage: list of instructions as _decode_words gives them."""
    words = sp.entries.cpu().numpy().view(np.uint32)
    ipc, ipc1 = sp.iters_per_chunk, sp.stage1_iters
    ng, R = sp.n // 8, sp.rows_per_chunk
    out = []
    for c in range(sp.n_chunks):
        stages = []
        for a, b in ((c * ipc, c * ipc + ipc1), (c * ipc + ipc1, (c + 1) * ipc)):
            stages.append(_decode_words(words[a * ITER_WORDS:b * ITER_WORDS], ng, R))
        out.append(stages)
    return out


@pytest.mark.parametrize("rows,n,bpw,R", [(300, 2048, 2, None), (256, 2048, 4, None), (100, 6144, 4, None),
                                          (1000, 512, 2, None), (97, 800, 2, None), (5, 64, 4, None),
                                          (1, 2048, 2, None), (3, 16, 2, None), (200, 2048, 3, None),
                                          (7, 16, 3, None),
                                          # taller chunks, 17-bit positions (bit 16 in the high byte)
                                          (700, 2048, 2, 350), (600, 2048, 4, 300), (300, 6144, 4, 120),
                                          (520, 512, 3, 511), (300, 2048, 3, 300),
                                          # short chunks: four 16-lane groups per instruction
                                          (300, 2048, 2, 16), (200, 2048, 4, 31), (97, 800, 3, 32),
                                          (64, 1024, 2, 5)])
def test_sorted_pack_is_a_permutation_with_distinct_rows(rows, n, bpw, R):
    ng = n // 8
    m = synth.vq_matrix(9800 + rows + bpw, rows, n, bpw=bpw)
    sp = SortedPlanes(m["idx0"], m["idx1"], rows, n, device="cpu", threads=3, rows_per_chunk=R)
    gb = _gb(ng)
    if R is None:  # the default chunking: 16-bit positions, at most 255 rows
        R = int(_lib.load().vq2_sorted_rows_per_chunk(rows, ng, 1))
        assert (R + 1) * (1 << gb) <= 1 << 16 and _pb(ng, R) <= 16 and R <= 255
    else:
        assert _pb(ng, R) == 17 or R == 511 or R <= 32
    assert sp.rows_per_chunk == R and sp.n_chunks == -(-rows // R)
    if sp.rows_per_chunk == int(_lib.load().vq2_sorted_rows_per_chunk(rows, ng, 1)):
        assert R * sp.n_chunks - rows < sp.n_chunks  # the default: the rows split evenly over the chunks
    assert rows // sp.n_chunks + (1 if rows % sp.n_chunks else 0) <= R
    assert sp.n_iters == sp.n_chunks * sp.iters_per_chunk                 # chunks padded to one size
    assert sp.entries.numel() == sp.n_iters * ITER_WORDS
    assert 0 < sp.stage1_iters <= sp.iters_per_chunk
    assert (sp.stage1_iters < sp.iters_per_chunk) == (bpw > 2)
    assert sp.s2_kind == {2: 0, 3: 2, 4: 1}[bpw]
    planes = [m["idx0"].numpy().view(np.uint16)]
    if bpw == 4:
        planes.append(m["idx1"].numpy().view(np.uint16))
    if bpw == 3:  # the (16,8) uint8 plane: packed as codes 0..255
        planes.append(m["idx1"].numpy().astype(np.uint16))
    dummy = R << gb
    for c, stages in enumerate(_decode(sp)):
        rb, nbig = rows // sp.n_chunks, rows % sp.n_chunks    # near-equal chunks: heights rb + 1 then rb
        r0 = c * rb + min(c, nbig)
        r1 = r0 + rb + (1 if c < nbig else 0)
        for st, instrs in enumerate(stages):
            if st >= len(planes):
                assert not instrs
                continue
            assert len(instrs) % 4 == 0
            codes = np.concatenate([i[0] for i in instrs])
            pos = np.concatenate([i[1] for i in instrs])
            real = pos != dummy
            assert np.all(np.concatenate([i[3] for i in instrs])[~real] == 0)  # padding: offset 0
            code, p = codes[real], pos[real]
            r, g = p >> gb, p & ((1 << gb) - 1)
            assert np.all(r < r1 - r0) and np.all(g < ng)
            got = np.zeros((r1 - r0, ng), np.int64) - 1
            assert len(code) == (r1 - r0) * ng          # every code exactly once ...
            got[r, g] = code
            assert np.array_equal(got, planes[st][r0:r1].astype(np.int64))  # ... at its row and group
            for cd, ps, base, off in instrs:
                rl = ps != dummy
                if rl.any():
                    assert base == cd[rl].min()           # the base is the instruction's smallest code
                # no row twice in a lane group (lane 63: the base): 32-lane
                # halves, or 16-lane quarters for chunks of at most 32 rows
                pl = 16 if R <= 32 else 32
                for lo in range(0, 64, pl):
                    hi = min(lo + pl, 63)
                    rr = ps[lo:hi][ps[lo:hi] != dummy] >> gb
                    assert len(np.unique(rr)) == len(rr)


def test_sorted_pack_keeps_instructions_within_few_lines():
    """At the gate/up shape (6144 x 2048, 4 bpw) a 63-code instruction of a
    246-row chunk (~63000 codes) spans ~8-10 128-byte codebook lines (8 fp16
    centroids per line) instead of the ~64 of unsorted codes; lane 63 gathers
    the base code's line, which lane 0 reads too."""
    rows, n = 6144, 2048
    m = synth.vq_matrix(9900, rows, n, bpw=4)
    sp = SortedPlanes(m["idx0"], m["idx1"], rows, n, device="cpu")
    dummy = sp.rows_per_chunk << _gb(n // 8)
    lines = []
    for stages in _decode(sp)[:8]:
        for instrs in stages:
            for cd, ps, base, off in instrs:
                if np.all(ps != dummy):
                    lines.append(len(np.unique(np.append(cd, base) >> 3)))
    assert 6 <= np.mean(lines) <= 12, np.mean(lines)
    print("mean codebook lines per instruction:", np.mean(lines))
    assert sp.n_iters <= 1.02 * (rows * n // 8 * 2) / 252  # little padding
    assert sp.entries.numel() * 4 <= 3.1 * rows * n // 8 * 2  # ~3 bytes per code


def test_sorted_pack_rejects_bad_input():
    m = synth.vq_matrix(9910, 16, 512, bpw=3)
    with pytest.raises(Vq2Error):
        SortedPlanes(m["idx0"], m["idx1"][:8], 16, 512, device="cpu")  # stage-2 plane of another size
    with pytest.raises(Vq2Error):
        SortedPlanes(m["idx0"], None, 17, 512, device="cpu")      # wrong row count
    L = _lib.load()
    n_it, ipc, ipc1 = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
    buf = torch.empty(ITER_WORDS, dtype=torch.int32)
    st = L.vq2_sorted_pack(m["idx0"].data_ptr(), None, 16, 64, 16, buf.data_ptr(), 1, ctypes.byref(ipc),
                           ctypes.byref(ipc1), ctypes.byref(n_it), 1)
    assert st == _lib.ERR_ARG and n_it.value > 1   # capacity too small: the needed size is reported
    assert n_it.value == ipc.value and ipc1.value == ipc.value
    st = L.vq2_sorted_pack(m["idx0"].data_ptr(), None, 16, 64, 512, buf.data_ptr(), 1000, ctypes.byref(ipc),
                           ctypes.byref(ipc1), ctypes.byref(n_it), 1)
    assert st == _lib.ERR_ARG                     # rows_per_chunk beyond 511
    st = L.vq2_sorted_pack(m["idx0"].data_ptr(), None, 16, 2048, 64, buf.data_ptr(), 1000, ctypes.byref(ipc),
                           ctypes.byref(ipc1), ctypes.byref(n_it), 1)
    assert st == _lib.ERR_ARG                     # ng 2048: 64 rows need an 18-bit position


def test_sorted_rows_per_chunk_alignment():
    L = _lib.load()
    # the LM head: 512 chunks of <= 297 rows (17-bit positions), one round
    # of two workgroups per CU, instead of 768 of 198 with 16-bit positions
    assert L.vq2_sorted_rows_per_chunk(151936, 256, 256) == 297
    assert L.vq2_sorted_rows_per_chunk(151936, 256, 1) == 255     # 596 chunks (no alignment asked)
    assert L.vq2_sorted_rows_per_chunk(100000, 256, 256) == 196   # 512 chunks, 16-bit positions suffice
    # fewer than 2^20 codes, packed for a launch of its own: about 0.75 x 256
    # chunks (ceil(4 rows / 768) rows each, at most 64)
    assert L.vq2_sorted_rows_per_chunk(2048, 256, 256) == 11      # o: 187 chunks
    assert L.vq2_sorted_rows_per_chunk(512, 256, 256) == 3        # k or v alone: 171 chunks
    assert L.vq2_sorted_rows_per_chunk(65536, 8, 256) == 64       # 0.5 M codes, capped at 64 rows
    assert L.vq2_sorted_rows_per_chunk(2048, 256, 1) == 228       # no alignment asked (expert pools): 9 chunks
    assert L.vq2_sorted_rows_per_chunk(6144, 256, 256) == 246     # 25 chunks (aligned ones would be too short)
    assert L.vq2_sorted_rows_per_chunk(2048, 768, 1) == 63        # 6144-wide: 63 rows at most (33 chunks)
    assert L.vq2_sorted_rows_per_chunk(100, 1 << 16, 1) == 0      # n beyond the 16-bit position field


@pytest.mark.parametrize("E,rows,n,R", [(3, 1024, 2048, None), (5, 2048, 512, None), (2, 100, 800, None),
                                         (3, 2048, 512, 410)])
def test_sorted_pool_pack_equals_per_expert_pack(E, rows, n, R):
    """vq2_sorted_pack_pool lays the experts out one after another, each
    chunk exactly as vq2_sorted_pack packs it alone (chunks of more than 32
    rows, where both deal into 32-lane halves), then padded with dummy-row
    iterations (offset 0, base code 0) to the pool's common iteration
    count.  Also for a taller pool (the MoE down pool in 5 chunks of 410
    rows, 16-bit positions)."""
    from compressai_amd.kernels import SortedPool

    ng = n // 8
    idx = synth.indices16(9950 + rows, (E, rows, ng))
    pool = SortedPool(idx, device="cpu", threads=3, rows_per_chunk=R)
    C, want = pool.chunks, R
    R = pool.rows_per_chunk
    assert R == (want or int(_lib.load().vq2_sorted_rows_per_chunk(rows, ng, 1))) and C == -(-rows // R)
    ipc = pool.iters_per_chunk
    assert pool.n_iters == E * C * ipc
    ent = pool.entries.numpy().view(np.uint32)
    pad = np.uint32(R << _gb(ng))
    pad_lane = np.array([pad | (pad << 16), pad | (pad << 16), 0], np.uint32)
    longest = 0
    W = ITER_WORDS
    for e in range(E):
        sp = SortedPlanes(idx[e], None, rows, n, device="cpu", chunk_align=1, rows_per_chunk=R)
        assert sp.rows_per_chunk == R and sp.n_chunks == C
        ipe = sp.iters_per_chunk   # this expert's chunks, padded to its own longest
        own = sp.entries.numpy().view(np.uint32)
        longest = max(longest, ipe)
        for c in range(C):
            got = ent[(e * C + c) * ipc * W:(e * C + c + 1) * ipc * W]
            assert np.array_equal(got[: ipe * W], own[c * ipe * W:(c + 1) * ipe * W])
            tail = got[ipe * W:].reshape(-1, 64, 3)
            assert np.all(tail[:, :63] == pad_lane) and np.all(tail[:, 63] == 0)
    assert ipc == longest


def test_sorted_pool_chunk_height_limits():
    """Pools keep 16-bit positions: up to 511 rows where ceil(log2 ng) leaves
    room (ng 64: 1023 would fit, 511 is the kernels' limit), 255 at ng 256;
    the taller down pool's height rule (moe._tall_rows) stays within it."""
    from compressai_amd.kernels import SortedPool
    from compressai_amd.moe import _tall_rows

    idx = synth.indices16(9960, (1, 600, 64))
    assert SortedPool(idx, device="cpu", rows_per_chunk=511).chunks == 2
    with pytest.raises(Vq2Error, match="rows_per_chunk=512"):
        SortedPool(idx, device="cpu", rows_per_chunk=512)
    idx = synth.indices16(9961, (1, 300, 256))
    assert SortedPool(idx, device="cpu", rows_per_chunk=255).chunks == 2
    with pytest.raises(Vq2Error, match="rows_per_chunk=256"):
        SortedPool(idx, device="cpu", rows_per_chunk=256)
    assert _tall_rows(2048, 64, 228) == 410       # the 35B down pool: 5 chunks instead of 9
    assert _tall_rows(1024, 256, 205) is None     # gate_up: 255 rows at most, 205 already
    assert _tall_rows(7168, 256, 240) is None     # 248 rows: not a quarter taller
    assert _tall_rows(4096, 128, 228) == 456      # ng 128: 511 rows at most, 9 chunks


def test_moe_slices_cost_model():
    """Slice counts of the sorted MoE launches on 256 CUs: T = 1 fills one
    round (gate_up 45 units x 5, down 81 x 3); T = 8 takes 2 and 1.  In the
    one launch (two workgroups per CU) units that fill the CUs take 2 slices
    and units that fill them twice 1; fewer follow the model."""
    from compressai_amd.kernels import moe_slices

    assert moe_slices(45, 205 * 256, 256, 2.5) == 5
    assert moe_slices(81, 228 * 64, 256, 2.0) == 3
    assert moe_slices(360, 205 * 256, 256, 2.5) == 2
    assert moe_slices(648, 228 * 64, 256, 2.0) == 1
    assert moe_slices(45, 205 * 256, 256, 2.5, one_launch=True) == 5
    assert moe_slices(81, 228 * 64, 256, 2.0, one_launch=True) == 3
    assert moe_slices(360, 205 * 256, 256, 2.5, one_launch=True) == 2
    assert moe_slices(648, 228 * 64, 256, 2.0, one_launch=True) == 1


@pytest.mark.parametrize("s2", ["u8", "i16"])
def test_sorted_two_stage_pool_equals_per_expert_pack(s2):
    """A two-stage pool ((16,8) uint8 or (16,16) int16 stage 2): every chunk
    holds the expert's stage-1 iterations as vq2_sorted_pack packs them,
    padded to the pool's stage-1 count, then its stage-2 iterations, padded
    to the pool's stage-2 count."""
    from compressai_amd.kernels import SortedPool

    E, rows, n = 3, 300, 512
    ng = n // 8
    idx = synth.indices16(9960, (E, rows, ng))
    if s2 == "u8":
        idx1 = torch.randint(0, 256, (E, rows, ng), generator=synth.gen(9961), dtype=torch.int32).to(torch.uint8)
    else:
        idx1 = synth.indices16(9961, (E, rows, ng))
    pool = SortedPool(idx, device="cpu", threads=2, idx1=idx1)
    assert pool.s2_kind == (2 if s2 == "u8" else 1)
    C, R, ipc, ipc1 = pool.chunks, pool.rows_per_chunk, pool.iters_per_chunk, pool.stage1_iters
    assert 0 < ipc1 < ipc and pool.n_iters == E * C * ipc
    W = ITER_WORDS
    ent = pool.entries.numpy().view(np.uint32)
    pad = np.uint32(R << _gb(ng))
    pad_lane = np.array([pad | (pad << 16), pad | (pad << 16), 0], np.uint32)

    def is_pad(words):
        t = words.reshape(-1, 64, 3)
        return np.all(t[:, :63] == pad_lane) and np.all(t[:, 63] == 0)

    for e in range(E):
        sp = SortedPlanes(idx[e], idx1[e], rows, n, device="cpu", chunk_align=1)
        own = sp.entries.numpy().view(np.uint32)
        ie, ie1 = sp.iters_per_chunk, sp.stage1_iters
        for c in range(C):
            got = ent[(e * C + c) * ipc * W:(e * C + c + 1) * ipc * W]
            o1 = own[c * ie * W:(c * ie + ie1) * W]
            o2 = own[(c * ie + ie1) * W:(c + 1) * ie * W]
            g1, g2 = got[:ipc1 * W], got[ipc1 * W:]
            assert np.array_equal(g1[:len(o1)], o1) and is_pad(g1[len(o1):])
            assert np.array_equal(g2[:len(o2)], o2) and is_pad(g2[len(o2):])
    empty = SortedPool.slots(pool, 5)
    assert empty.n_iters == 5 * C * ipc and empty.stage1_iters == ipc1 and int(empty.entries.abs().sum()) == 0
