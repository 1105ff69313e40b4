"""Host-side checks that need no GPU: launch validation of the Python entry
points, the reference CPU path restated in oracle/ref_cpu_path.py (the timed
CPU baseline) against the C oracle, the oracle's top-1 against numpy, the
rotation tables against the committed golden fixture, and the drop-in
modules' constructors."""
import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from compressai_amd import synth
from compressai_amd.kernels import Vq2Error, check_gemv_rht_mats
from compressai_amd.rot import rot_tables, tag_seed
from oracle import ref_cpu_path as R
from oracle import vq2_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "rot_tables.npz"


# ------------------------------------------------- launch validation (CPU)
def _mat(rows, n, s2=None, sdt=torch.float16, seed=0):
    g = torch.Generator().manual_seed(seed)
    i0 = torch.randint(-32768, 32768, (rows, n // 8), generator=g, dtype=torch.int32).to(torch.int16)
    i1 = None
    if s2 == "u8":
        i1 = torch.randint(0, 256, (rows, n // 8), generator=g, dtype=torch.int32).to(torch.uint8)
    elif s2 == "u16":
        i1 = torch.randint(-32768, 32768, (rows, n // 8), generator=g, dtype=torch.int32).to(torch.int16)
    return (i0, i1, (torch.rand(rows, generator=g) + 0.5).to(sdt), rows)


def test_gemv_rht_checks_accept_consistent_launch():
    cb0 = torch.zeros(65536, 8, dtype=torch.float16)
    cb1 = torch.zeros(65536, 8, dtype=torch.float16)
    s2, mats = check_gemv_rht_mats([_mat(64, 256, "u16"), _mat(32, 256, "u16")], cb0, cb1, 256)
    assert s2 == 2 and [m[3] for m in mats] == [64, 32]


@pytest.mark.parametrize("case", ["u16_then_u8", "u8_then_u16", "none_then_u16", "scale_dtype_mix",
                                  "short_cb0", "short_cb1_u16", "missing_cb1", "cb_dtype_mix", "bad_rows",
                                  "too_many"])
def test_gemv_rht_checks_reject_mixes(case):
    """Every matrix of a vq_gemv_rht launch is checked, not only the first
    or the last: a mix the single launch cannot express raises Vq2Error
    before anything reaches the device."""
    n = 256
    cb0 = torch.zeros(65536, 8, dtype=torch.float16)
    cb1 = torch.zeros(65536, 8, dtype=torch.float16)
    cb8 = torch.zeros(256, 8, dtype=torch.float16)
    mats, c1 = None, cb1
    if case == "u16_then_u8":
        mats = [_mat(64, n, "u16"), _mat(64, n, "u8")]
    elif case == "u8_then_u16":
        mats, c1 = [_mat(64, n, "u8"), _mat(64, n, "u16")], cb8
    elif case == "none_then_u16":
        mats = [_mat(64, n), _mat(64, n, "u16")]
    elif case == "scale_dtype_mix":
        mats = [_mat(64, n, sdt=torch.float32), _mat(64, n, sdt=torch.float16), _mat(64, n, sdt=torch.float32)]
    elif case == "short_cb0":
        mats, cb0 = [_mat(64, n)], torch.zeros(4096, 8, dtype=torch.float16)
    elif case == "short_cb1_u16":
        mats, c1 = [_mat(64, n, "u16")], cb8
    elif case == "missing_cb1":
        mats, c1 = [_mat(64, n, "u8")], None
    elif case == "cb_dtype_mix":
        mats, c1 = [_mat(64, n, "u16")], cb1.to(torch.bfloat16)
    elif case == "bad_rows":
        i0, i1, s, r = _mat(64, n)
        mats = [(i0, i1, s, 63)]
    elif case == "too_many":
        mats = [_mat(8, n) for _ in range(5)]
    with pytest.raises(Vq2Error):
        check_gemv_rht_mats(mats, cb0, c1, n)


# --------------------------------------------- reference CPU path (baseline)
def test_cpu_moe_twins_match_oracle():
    """vq_moe_parallel_gate_up_cpu / _down_cpu restated (fp32 codebook, as
    the reference's CPU test feeds them) against the C oracle's grouped GEMV."""
    E, OUT, NG = 5, 96, 32
    cb = synth.codebook(8100).float()
    pool = synth.indices16(8101, (E, OUT, NG))
    ps = synth.scales(8102, (E, OUT))
    slots = [3, 0, 3, 4]
    x = synth.activations(8103, NG * 8, dtype=torch.float32)
    y = R.moe_gate_up_cpu(x, slots, pool, cb, ps, OUT=OUT, NG=NG, rs=0.5)
    _, y64 = O.moe_grouped(x, np.array(slots, np.int32), pool, cb, ps, OUT, NG, rs=0.5)
    assert O.max_rel_err(y.numpy(), y64) < 1e-5
    act = synth.activations(8104, (len(slots), NG * 8), dtype=torch.float32)
    yd = R.moe_down_cpu(act, slots, pool, cb, ps, OUT=OUT, NG=NG)
    _, yd64 = O.moe_grouped(act, np.array(slots, np.int32), pool, cb, ps, OUT, NG, per_pair_x=True)
    assert O.max_rel_err(yd.numpy(), yd64) < 1e-5


def test_cpu_moe_layer_matches_oracle():
    """The restated MoE layer (router, shared expert, per-token loop) against
    the fp64 oracle's layer, T = 3, 12 routed experts + 1 shared, top-4."""
    E, k, T, H, I = 12, 4, 3, 2048, 512
    cb = synth.codebook(8200)
    gu = synth.indices16(8202, (E + 1, 2 * I, H // 8))
    gus = synth.scales(8203, (E + 1, 2 * I))
    dn = synth.indices16(8212, (E + 1, H, I // 8))
    dns = synth.scales(8213, (E + 1, H))
    h = synth.activations(8204, (T, H))
    logits = synth.activations(8207, (T, E))
    gate = synth.activations(8208, H) * 0.02
    ph, sh = synth.permutation(8205, H), synth.signs(8206, H)
    pi, si = synth.permutation(8215, I), synth.signs(8216, I)
    out = R.moe_layer_cpu(h, logits, cb.float(), gu, gus, dn, dns, gate, R.CpuRot(ph, sh, 2048),
                          R.CpuRot(pi, si, 512), top_k=k, shared_id=E)
    ref = O.moe_layer(h, logits, cb, gu[:E].numpy(), gus[:E], dn[:E].numpy(), dns[:E], gu[E].numpy(), gus[E],
                      dn[E].numpy(), dns[E], gate, ph.numpy(), sh.float().numpy(), pi.numpy(), si.float().numpy(),
                      top_k=k)
    assert O.max_rel_err(out.numpy(), ref) < 1e-4


@pytest.mark.parametrize("bpw,n", [(2, 2048), (3, 2048), (4, 6144)])
def test_cpu_packed_linear_fallback_matches_oracle(bpw, n):
    """The restated PackedLinear fp32 fallback (RHT, dequant, F.linear)
    against the C oracle's RHT + VQ GEMV."""
    out = 256
    cb0 = synth.codebook(8300)
    cb1 = synth.codebook(8301, 256 if bpw == 3 else 65536) if bpw > 2 else None
    m = synth.vq_matrix(8300 + n + bpw, out, n, bpw=bpw)
    x = synth.activations(8304, (2, n))
    perm, sign = synth.permutation(8305, n), synth.signs(8306, n)
    y = R.packed_linear_fallback(x, R.CpuRot(perm, sign, 2048), m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    xr = O.rht(x, perm, sign, 2048)
    _, y64 = O.vq_gemv(xr.astype(np.float32), m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert O.max_rel_err(y.numpy(), y64) < 1e-5


# ----------------------------------------------------------- top-1 oracle
def test_oracle_argmax_matches_numpy():
    """orc_argmax_rows is numpy.argmax (first maximum), ties included."""
    g = np.random.default_rng(8400)
    v = g.standard_normal((7, 5000))
    v[2, 100] = v[2, 4000] = v[2].max() + 1.0      # tie: the first index wins
    v[5, :] = 0.0                                  # all equal: index 0
    v[6, 4999] = 1e30                               # the last column
    assert O.argmax_rows(v).tolist() == np.argmax(v, axis=1).tolist()
    assert O.argmax_rows(v)[2] == 100 and O.argmax_rows(v)[5] == 0 and O.argmax_rows(v)[6] == 4999


# ----------------------------------------------------- rotation fixtures
def test_rot_tables_match_golden_fixture():
    """Rot's perm / sign draws (md5 seed -> randperm -> randint) equal the
    committed fixture written by tests/golden/make_rot_tables.py."""
    G = np.load(GOLDEN)
    tags = sorted({k.rsplit("|", 2)[0] + "|" + k.rsplit("|", 2)[1] for k in G.files})
    assert len(tags) == 3
    for key in tags:
        tag, n = key.split("|")
        n = int(n)
        assert int(G[f"{key}|seed"][0]) == tag_seed(tag) == int(hashlib.md5(tag.encode()).hexdigest()[:8], 16)
        perm, sign = rot_tables(n, tag_seed(tag))
        assert np.array_equal(perm.numpy(), G[f"{key}|perm"].astype(np.int64)), tag
        assert np.array_equal(sign.numpy(), G[f"{key}|sign"].astype(np.float32)), tag


# ------------------------------------------------ drop-in constructors
def test_packed_linear_holds_bf16_scales():
    """PackedLinear rounds the row scales to bf16 at construction, as the
    reference does (vq2/runtime.py:78); scale_dtype=None keeps them."""
    from compressai_amd.runtime import PackedLinear

    m = synth.vq_matrix(8500, 64, 512, bpw=2)
    cbs = {"16": synth.codebook(8500)}
    lin = PackedLinear((64, 512), (16,), "t", [m["idx0"]], m["scale"], cbs, "cpu")
    assert lin.scale.dtype == torch.bfloat16 and torch.equal(lin.scale, m["scale"].to(torch.bfloat16))
    keep = PackedLinear((64, 512), (16,), "t", [m["idx0"]], m["scale"], cbs, "cpu", scale_dtype=None)
    assert keep.scale.dtype == torch.float16 and torch.equal(keep.scale, m["scale"])


def test_packed_linear_release_planes_needs_a_sorted_copy():
    """release_planes() keeps the planes of a module without a code-sorted
    copy (here: on the CPU, where none is built) and says why."""
    from compressai_amd.kernels import Vq2Error
    from compressai_amd.runtime import PackedLinear

    m = synth.vq_matrix(8501, 64, 512, bpw=2)
    lin = PackedLinear((64, 512), (16,), "t", [m["idx0"]], m["scale"], {"16": synth.codebook(8501)}, "cpu")
    assert lin.sorted is None and not lin.planes_released
    with pytest.raises(Vq2Error, match="no code-sorted copy"):
        lin.release_planes()
    assert torch.equal(lin.idx0, m["idx0"])


def test_resident_experts_reference_constructor_on_cpu():
    """ResidentMoEExperts(q_gate_up, q_down, cb16, device): the quantized
    dicts are viewed as [E, 2I, H/8] / [E, H, I/8] pools with bf16 scales
    (vq2/load_and_test_full_35b.py:37-40); wrong sizes raise."""
    from compressai_amd.moe import PackedMoEExpertUniversal, ResidentMoEExperts

    E, H, I = 4, 512, 128
    gu = synth.indices16(8600, (E * 2 * I, H // 8))
    dn = synth.indices16(8601, (E * H, I // 8))
    q_gu = {"idx": [gu], "scale": synth.scales(8602, E * 2 * I), "cfg": (16,)}
    q_dn = {"idx": [dn], "scale": synth.scales(8603, E * H), "cfg": (16,)}
    cb = synth.codebook(8604)
    mod = PackedMoEExpertUniversal(q_gu, q_dn, cb, "cpu", num_experts=E, hidden_dim=H, intermediate_dim=I)
    assert isinstance(mod, ResidentMoEExperts)
    assert mod.gate_up_idx.shape == (E, 2 * I, H // 8) and mod.down_idx.shape == (E, H, I // 8)
    assert torch.equal(mod.gate_up_idx.reshape(-1), gu.reshape(-1))
    assert mod.gate_up_scale.dtype == torch.bfloat16 and mod.down_scale.dtype == torch.bfloat16
    assert torch.equal(mod.down_scale, q_dn["scale"].view(E, H).to(torch.bfloat16))
    with pytest.raises(Vq2Error):
        ResidentMoEExperts(q_gu, q_dn, cb, "cpu", num_experts=E + 1, hidden_dim=H, intermediate_dim=I)


def test_resident_experts_tall_down_pool_on_cpu():
    """The sorted layout keeps the down pool twice at the 35B shape: 9 chunks
    of 228 rows for T = 1 and 5 of 410 for T >= 2; both count in nbytes(),
    and release_tall_down() returns every T to the default chunks."""
    from compressai_amd.moe import ResidentMoEExperts

    E, H, I = 2, 2048, 512
    gu = synth.indices16(8610, (E, 2 * I, H // 8))
    dn = synth.indices16(8611, (E, H, I // 8))
    mod = ResidentMoEExperts.from_pools(gu, synth.scales(8612, (E, 2 * I)), dn, synth.scales(8613, (E, H)),
                                        synth.codebook(8614), sorted_layout=True)
    d, t = mod.sorted_dn, mod.sorted_dn_tall
    assert (d.rows_per_chunk, d.chunks) == (228, 9) and (t.rows_per_chunk, t.chunks) == (410, 5)
    assert mod._down_pool(1) is d and mod._down_pool(2) is t and mod._down_pool(64) is t
    full = mod.nbytes()
    mod.release_tall_down()
    assert mod.sorted_dn_tall is None and mod._down_pool(8) is d and full - mod.nbytes() == t.nbytes()
    plain = ResidentMoEExperts.from_pools(gu, synth.scales(8612, (E, 2 * I)), dn, synth.scales(8613, (E, H)),
                                          synth.codebook(8614), sorted_layout=False)
    assert plain.sorted_dn is None and plain.sorted_dn_tall is None


# ---------------------------------- vq_sorted_moe argument checks (CPU)
def _small_sorted_pools():
    from compressai_amd.kernels import SortedPool

    E, H, I = 2, 64, 32
    gu = SortedPool(synth.indices16(7100, (E, 2 * I, H // 8)), device="cpu", threads=1)
    dn = SortedPool(synth.indices16(7101, (E, H, I // 8)), device="cpu", threads=1)
    return E, H, I, gu, dn


def _rot(n, perm_dt=torch.int32, sign_dt=torch.int8, n_perm=None, n_sign=None):
    perm = torch.arange(n if n_perm is None else n_perm, dtype=perm_dt)
    sign = torch.ones(n if n_sign is None else n_sign, dtype=sign_dt)
    return (perm, sign, n, n ** -0.5)


@pytest.mark.parametrize("which,bad", [
    ("rot_h", dict(n_perm=63)), ("rot_h", dict(perm_dt=torch.int64)), ("rot_h", dict(n_sign=65)),
    ("rot_h", dict(sign_dt=torch.int32)), ("rot_i", dict(n_perm=31)), ("rot_i", dict(sign_dt=torch.float32)),
    ("rot_i", dict(n_sign=64)),
])
def test_sorted_moe_rejects_bad_rotation_tables(which, bad):
    """Each rotation table is read over H (rot_h) or I (rot_i) entries by the
    kernels: a short, long or wrong-dtype table is refused on the host."""
    from compressai_amd.kernels import vq_sorted_moe

    E, H, I, gu, dn = _small_sorted_pools()
    rh = _rot(H, **bad) if which == "rot_h" else _rot(H)
    ri = _rot(I, **bad) if which == "rot_i" else _rot(I)
    with pytest.raises(Vq2Error, match=which):
        vq_sorted_moe(torch.zeros(1, H), gu, torch.ones(E, 2 * I), dn, torch.ones(E, H),
                      torch.zeros(65536, 8, dtype=torch.float16), rh, ri,
                      ids=torch.zeros(1, 1, dtype=torch.int32), w=torch.ones(1, 1))


def test_sorted_moe_rejects_noncontiguous_table_and_bad_gate():
    from compressai_amd.kernels import vq_sorted_moe

    E, H, I, gu, dn = _small_sorted_pools()
    args = (torch.zeros(1, H), gu, torch.ones(E, 2 * I), dn, torch.ones(E, H),
            torch.zeros(65536, 8, dtype=torch.float16))
    perm = torch.arange(2 * H, dtype=torch.int32)[::2]  # H entries, strided
    with pytest.raises(Vq2Error, match="rot_h perm"):
        vq_sorted_moe(*args, (perm, None, H, 1.0), _rot(I), ids=torch.zeros(1, 1, dtype=torch.int32),
                      w=torch.ones(1, 1))
    router = dict(logits=torch.zeros(1, E - 1), top_k=1, shared_id=E - 1)
    for gate, msg in ((torch.zeros(H - 1), "shared_gate"), (torch.zeros(H, dtype=torch.int32), "shared_gate"),
                      (torch.zeros(2 * H)[::2], "shared_gate"), (None, "router needs")):
        with pytest.raises(Vq2Error, match=msg):
            vq_sorted_moe(*args, _rot(H), _rot(I), shared_gate=gate, **router)
