"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on
identical seeded inputs.

Tolerances (the decode-path contract):
  * index decode and dequantized weights: bit-exact;
  * fp32 outputs: max_i |y_i - ref_i| / max_i |ref_i| <= 1e-3 against the
    fp64-accumulation oracle (observed ~1e-6: fp32 accumulation in a
    different order);
  * bf16 outputs: within one bf16 ulp (2^-8 relative) of the oracle rounded
    to bf16 (the reference kernels store bf16);
  * RHT: <= 1e-5 (fp32 butterflies against fp64).
"""
import numpy as np
import pytest
import torch

from compressai_amd import kernels as K, synth
from oracle import vq2_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _cuda(*ts, dev):
    return [None if t is None else t.to(dev) for t in ts]


# --------------------------------------------------------------------- RHT
@pytest.mark.parametrize("hb,n,batch", [(2, 2, 1), (8, 16, 3), (64, 64, 2), (128, 256, 1), (256, 256, 5),
                                        (512, 512, 9), (1024, 1024, 1), (2048, 2048, 1), (2048, 6144, 2),
                                        (4096, 4096, 1), (8192, 8192, 2), (2048, 8192, 4)])
@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_rht_forward_vs_oracle(dev, hb, n, batch, dt):
    x = synth.activations(11 + n, (batch, n), dtype=dt)
    perm = synth.permutation(12 + n, n)
    sign = synth.signs(13 + n, n)
    y = K.vq_rht(x.to(dev), perm.to(dev), sign.to(dev), hb, out_dtype=torch.float32)
    ref = O.rht(x, perm, sign, hb)
    assert O.max_rel_err(y.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("offset", [0, 1])
def test_rht_forward_staged_and_unaligned_bad_perm(dev, dt, offset):
    """The forward permuted transform stages 16-byte aligned rows in LDS
    (offset 0) and gathers through the permutation otherwise (offset 1: rows
    start 1 element past alignment).  An out-of-range permutation entry
    poisons its block with NaN on both paths; the other blocks match the
    oracle."""
    n, hb, batch = 8192, 2048, 3
    flat = synth.activations(51, batch * n + 8, dtype=dt)
    xh = flat[offset:offset + batch * n].view(batch, n)
    x = flat.to(dev)[offset:offset + batch * n].view(batch, n)  # contiguous, storage offset `offset`
    perm = synth.permutation(52, n)
    sign = synth.signs(53, n)
    bad_slot = 5000  # block 2
    pbad = perm.clone()
    pbad[bad_slot] = n + 3
    y = K.vq_rht(x, pbad.to(dev), sign.to(dev), hb, out_dtype=torch.float32).cpu().numpy()
    ref = O.rht(xh.float(), perm, sign, hb)
    blk = bad_slot // hb
    assert np.all(np.isnan(y[:, blk * hb:(blk + 1) * hb]))
    keep = np.ones(n, dtype=bool)
    keep[blk * hb:(blk + 1) * hb] = False
    assert O.max_rel_err(y[:, keep], ref[:, keep]) < 1e-5


@pytest.mark.parametrize("hb,n", [(512, 512), (2048, 6144)])
def test_rht_inverse_roundtrip(dev, hb, n):
    x = synth.activations(21, (3, n), dtype=torch.float32).to(dev)
    perm = synth.permutation(22, n).to(dev)
    sign = synth.signs(23, n).to(dev)
    y = K.vq_rht(x, perm, sign, hb)
    z = K.vq_rht(y, perm, sign, hb, inverse=True)
    ref = O.rht(y.cpu(), perm.cpu(), sign.cpu(), hb, inverse=True)
    assert O.max_rel_err(z.cpu().numpy(), ref) < 1e-5
    assert torch.allclose(z, x, atol=1e-5)
    # orthogonality: norms preserved
    assert torch.allclose(y.norm(dim=1), x.norm(dim=1), rtol=1e-5)


def test_rht_no_perm_no_sign_and_bf16_in_out(dev):
    x = synth.activations(31, (2, 2048), dtype=torch.bfloat16)
    y = K.vq_rht(x.to(dev), None, None, 2048)  # bf16 out, like Rot.fwd on bf16
    assert y.dtype == torch.bfloat16
    ref = O.rht(x, None, None, 2048)
    refb = torch.from_numpy(ref.astype(np.float32)).to(torch.bfloat16).float().numpy()
    assert np.max(np.abs(y.float().cpu().numpy() - refb)) <= np.max(np.abs(refb)) * 2 ** -8


def test_swiglu_rht_vs_oracle(dev):
    I = 512
    gu = synth.activations(41, (9, 2 * I), dtype=torch.float32)
    perm = synth.permutation(42, I)
    sign = synth.signs(43, I)
    y = K.vq_swiglu_rht(gu.to(dev), I, perm.to(dev), sign.to(dev), 512)
    g = gu.double().numpy()
    act = g[:, :I] / (1 + np.exp(-g[:, :I])) * g[:, I:]
    ref = O.np_rht64(act, perm, sign, 512)
    assert O.max_rel_err(y.cpu().numpy(), ref) < 1e-5


# ---------------------------------------------------- dequant / decode exact
def test_decode_idx_exhaustive(dev):
    pat = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    got = K.vq_decode_idx(pat.to(dev)).cpu().numpy()
    assert np.array_equal(got, O.decode_idx16(pat.numpy()))
    u8 = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    assert K.vq_decode_idx(u8.to(dev)).cpu().tolist() == list(range(256))


@pytest.mark.parametrize("bpw", [2, 3, 4])
@pytest.mark.parametrize("cbdt", [torch.float16, torch.bfloat16, torch.float32])
def test_dequant_bitexact(dev, bpw, cbdt):
    cb0 = synth.codebook(51, dtype=cbdt)
    cb1 = synth.codebook(52, 256 if bpw == 3 else 65536, dtype=cbdt) if bpw > 2 else None
    m = synth.vq_matrix(5000, 96, 512, bpw=bpw)
    got = K.vq_dequant_rows(*_cuda(m["idx0"], m["idx1"], cb0, cb1, m["scale"], dev=dev), 5, 77).cpu().numpy()
    ref = O.dequant_rows(m["idx0"], m["idx1"], cb0, cb1, m["scale"], 5, 77)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# -------------------------------------------------------------------- GEMV
GEMV_CASES = [
    # (out, n, bpw, batch)
    (2048, 2048, 2, 1),    # config 1
    (512, 2048, 2, 1),     # config 2 k/v
    (6144, 2048, 4, 1),    # config 2 gate/up
    (2048, 6144, 4, 1),    # config 2 down (split-K over 3 waves)
    (2048, 2048, 3, 1),    # (16, 8) 3 bpw
    (1000, 2048, 2, 1),    # OUT not a multiple of any tile
    (7, 512, 2, 3),        # tiny, batch 3
    (333, 200, 2, 2),      # n/8 = 25: scalar (unaligned) index path
    (64, 8, 4, 1),         # n = 8: one group per row
    (1024, 2048, 2, 4),
    (257, 1024, 4, 5),     # batch tile 8 with 5 columns
    (512, 6144, 3, 8),
    (300, 4096, 2, 16),    # two batch tiles
    (96, 64 * 1024, 2, 1), # 32 K-chunks: waves loop over chunks
]


@pytest.mark.parametrize("out,n,bpw,batch", GEMV_CASES)
def test_gemv_fp32_vs_oracle(dev, out, n, bpw, batch):
    seed = 6000 + out + n + bpw
    cb0 = synth.codebook(seed)
    cb1 = synth.codebook(seed + 1, 256 if bpw == 3 else 65536) if bpw > 2 else None
    m = synth.vq_matrix(seed, out, n, bpw=bpw)
    x = synth.activations(seed + 4, (batch, n), dtype=torch.float32)
    y = K.vq_gemv(*_cuda(x, m["idx0"], m["idx1"], cb0, cb1, m["scale"], dev=dev), out, n, 0.5,
                  out_dtype=torch.float32)
    _, y64 = O.vq_gemv(x, m["idx0"], m["idx1"], cb0, cb1, m["scale"], rs=0.5)
    assert y.shape == (batch, out)
    assert O.max_rel_err(y.cpu().numpy(), y64) < TOL


@pytest.mark.parametrize("cbdt,xdt,sdt", [(torch.bfloat16, torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.float16, torch.float32),
                                          (torch.float16, torch.bfloat16, torch.float16)])
@pytest.mark.parametrize("bpw", [2, 3, 4])
def test_gemv_dtypes(dev, cbdt, xdt, sdt, bpw):
    cb0 = synth.codebook(71, dtype=cbdt)
    cb1 = synth.codebook(72, 256 if bpw == 3 else 65536, dtype=cbdt) if bpw > 2 else None
    m = synth.vq_matrix(7000, 384, 1024, bpw=bpw)
    sc = m["scale"].to(sdt)
    x = synth.activations(74, 1024, dtype=xdt)
    y = K.vq_gemv(*_cuda(x, m["idx0"], m["idx1"], cb0, cb1, sc, dev=dev), 384, 1024, 1.0, out_dtype=torch.float32)
    _, y64 = O.vq_gemv(x, m["idx0"], m["idx1"], cb0, cb1, sc)
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL


def test_gemv_drop_in_bf16_output(dev):
    """vq_gemv_16 / vq_gemv_16_8 keep the reference's bf16 output."""
    cb0 = synth.codebook(81, dtype=torch.bfloat16)
    cb1 = synth.codebook(82, 256, dtype=torch.bfloat16)
    m = synth.vq_matrix(8000, 2048, 2048, bpw=3)
    sc = m["scale"].to(torch.bfloat16)
    x = synth.activations(84, 2048, dtype=torch.bfloat16)
    xd, i0, i1, c0, c1, s = _cuda(x, m["idx0"], m["idx1"], cb0, cb1, sc, dev=dev)
    for y, (_, y64) in ((K.vq_gemv_16(xd, i0, c0, s, 2048, 2048, 2048 ** -0.5),
                         O.vq_gemv(x, m["idx0"], None, cb0, None, sc, rs=2048 ** -0.5)),
                        (K.vq_gemv_16_8(xd, i0, i1, c0, c1, s, 2048, 2048, 2048 ** -0.5),
                         O.vq_gemv(x, m["idx0"], m["idx1"], cb0, cb1, sc, rs=2048 ** -0.5))):
        assert y.dtype == torch.bfloat16 and y.shape == (2048,)
        ref = torch.from_numpy(y64[0].astype(np.float32)).to(torch.bfloat16).float().numpy()
        diff = np.abs(y.float().cpu().numpy() - ref)
        # at most one bf16 ulp of the value
        assert np.all(diff <= np.abs(ref) * 2 ** -7 + 1e-30)


def test_gemv_linearity_full_size(dev):
    """Size-independent property at the LM-head shape: y(2a - 3b) = 2y(a) - 3y(b)."""
    out, n = 151936, 2048
    cb = synth.codebook(91).to(dev)
    m = synth.vq_matrix(9000, out, n, bpw=2)
    i0, s = m["idx0"].to(dev), m["scale"].to(dev)
    a = synth.activations(94, n, dtype=torch.float32).to(dev)
    b = synth.activations(95, n, dtype=torch.float32).to(dev)
    f = lambda v: K.vq_gemv_16(v, i0, cb, s, out, n, out_dtype=torch.float32).double()
    lhs, rhs = f(2 * a - 3 * b), 2 * f(a) - 3 * f(b)
    assert ((lhs - rhs).abs().max() / rhs.abs().max()).item() < 1e-5


# ------------------------------------------------------------ LM head top-1
@pytest.mark.parametrize("batch", [1, 4])
def test_lm_head_argmax_full_size(dev, batch):
    """Config 3: 151936 x 2048 at 2 bpw, batch 1 and 4, fused top-1."""
    out, n = 151936, 2048
    cb = synth.codebook(3000)
    m = synth.vq_matrix(3000, out, n, bpw=2)
    x = synth.activations(3004, (batch, n), dtype=torch.float32)
    idx, val = K.vq_gemv_argmax(*_cuda(x, m["idx0"], None, cb, None, m["scale"], dev=dev), out, n)
    _, y64 = O.vq_gemv(x, m["idx0"], None, cb, None, m["scale"])
    ref = O.argmax_rows(y64)
    assert idx.cpu().tolist() == ref.tolist()
    # batch 4 takes the matrix-core path (fp16 activation, ~1e-4): the 1e-3 contract
    assert np.allclose(val.cpu().numpy(), y64[np.arange(batch), ref], rtol=1e-4 if batch < 3 else TOL)


def test_argmax_ties_pick_first(dev):
    v = torch.zeros(3, 50000)
    v[0, 17] = 5.0
    v[0, 40000] = 5.0
    v[1, :] = -1.0
    v[2, 49999] = 1.0
    v[2, 8192] = 1.0  # tie across argmax chunks
    idx, val = K.vq_argmax(v.to(dev))
    assert idx.cpu().tolist() == [17, 0, 8192]
    assert val.cpu().tolist() == [5.0, -1.0, 1.0]


# -------------------------------------------------------------- grouped MoE
def _pools(seed, E, dev=None):
    gu = synth.indices16(seed + 2, (E, 1024, 256))
    gus = synth.scales(seed + 3, (E, 1024))
    dn = synth.indices16(seed + 12, (E, 2048, 64))
    dns = synth.scales(seed + 13, (E, 2048))
    return gu, gus, dn, dns


@pytest.mark.parametrize("ids_dtype", [torch.int32, torch.int64])
def test_moe_parallel_gate_up_and_down_drop_in(dev, ids_dtype):
    """The reference call shapes: y_out written in place, bf16 pools/scales."""
    E = 12
    cb = synth.codebook(4000, dtype=torch.bfloat16)
    gu, gus, dn, dns = _pools(4000, E)
    gus, dns = gus.to(torch.bfloat16), dns.to(torch.bfloat16)
    ids = torch.tensor([3, 11, 0, 3, 7, 5, 9, 1], dtype=ids_dtype)
    xr = synth.activations(4004, 2048, dtype=torch.bfloat16)
    y_gu = torch.zeros(8, 1024, dtype=torch.float32, device=dev)
    K.vq_moe_parallel_gate_up(*_cuda(xr, ids, gu, cb, gus, dev=dev), y_gu, OUT=1024, NG=256, rs=0.7)
    _, ref = O.moe_grouped(xr, ids.numpy(), gu.numpy(), cb, gus, 1024, 256, rs=0.7)
    assert O.max_rel_err(y_gu.cpu().numpy(), ref) < TOL
    assert torch.equal(y_gu[0], y_gu[3])  # same expert, same row values

    act = synth.activations(4005, (8, 512), dtype=torch.bfloat16)
    y_dn = torch.empty(8, 2048, dtype=torch.bfloat16, device=dev)
    K.vq_moe_parallel_down(*_cuda(act, ids, dn, cb, dns, dev=dev), y_dn, OUT=2048, NG=64)
    _, ref = O.moe_grouped(act, ids.numpy(), dn.numpy(), cb, dns, 2048, 64, per_pair_x=True)
    refb = torch.from_numpy(ref.astype(np.float32)).to(torch.bfloat16).float().numpy()
    diff = np.abs(y_dn.float().cpu().numpy() - refb)
    assert np.all(diff <= np.abs(refb) * 2 ** -7 + 1e-30)


def test_moe_bad_expert_id_gives_nan_rows(dev):
    E = 4
    cb = synth.codebook(4100)
    gu, gus, _, _ = _pools(4100, E)
    ids = torch.tensor([1, E, -1, 2], dtype=torch.int32)
    xr = synth.activations(4104, 2048, dtype=torch.float32)
    y = torch.zeros(4, 1024, device=dev)
    K.vq_moe_parallel_gate_up(*_cuda(xr, ids, gu, cb, gus, dev=dev), y)
    yc = y.cpu()
    assert torch.isnan(yc[1]).all() and torch.isnan(yc[2]).all()
    assert not torch.isnan(yc[0]).any() and not torch.isnan(yc[3]).any()


def test_moe_down_combine_vs_oracle(dev):
    E, T, P = 10, 3, 5
    cb = synth.codebook(4200)
    _, _, dn, dns = _pools(4200, E)
    ids = torch.randint(0, E, (T, P), generator=synth.gen(4201), dtype=torch.int32)
    w = torch.rand(T, P, generator=synth.gen(4202))
    act = synth.activations(4203, (T * P, 512), dtype=torch.float32)
    out = K.vq_moe_down_combine(*_cuda(act, ids, w, dn, cb, dns, dev=dev), OUT=2048, NG=64)
    _, y = O.moe_grouped(act, ids.reshape(-1).numpy(), dn.numpy(), cb, dns, 2048, 64, per_pair_x=True)
    ref = (y.reshape(T, P, 2048) * w.double().numpy()[:, :, None]).sum(1)
    assert O.max_rel_err(out.cpu().numpy(), ref) < TOL


def test_router_topk_vs_oracle(dev):
    T, E, k = 8, 256, 8
    logits = synth.activations(4307, (T, E))
    h = synth.activations(4304, (T, 2048))
    gate = synth.activations(4308, 2048) * 0.02
    ids, w = K.vq_router_topk(*_cuda(logits, dev=dev), k, h.to(dev), gate.to(dev), shared_id=E)
    rid, rw = O.router_topk(logits, k)
    assert ids[:, :k].cpu().numpy().tolist() == rid.tolist()
    assert np.allclose(w[:, :k].cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    assert (ids[:, k] == E).all()
    sg = 1 / (1 + np.exp(-(h.double().numpy() @ gate.double().numpy())))
    assert np.allclose(w[:, k].cpu().numpy(), sg, rtol=1e-5)


@pytest.mark.parametrize("sorted_layout", [True, False])
@pytest.mark.parametrize("T", [1, 8])
def test_moe_layer_config4_vs_oracle(dev, T, sorted_layout):
    """Config 4: 256 routed + 1 shared expert resident in one pool, top-8,
    T = 1 and 8, router + RHTs + grouped GEMVs + combine on device, over the
    code-sorted pools and over the reference pools (gather kernels)."""
    from compressai_amd.moe import MoELayer

    E, k = 256, 8
    cb = synth.codebook(4000)
    gu, gus, dn, dns = _pools(4000, E + 1)
    h = synth.activations(4004, (T, 2048))
    logits = synth.activations(4007, (T, E))
    gate = synth.activations(4008, 2048) * 0.02
    layer = MoELayer(*_cuda(gu, gus, dn, dns, cb, gate, dev=dev), top_k=k, sorted_layout=sorted_layout)
    assert (layer.experts_mod.sorted_gu is not None) == sorted_layout
    out = layer(h.to(dev), logits.to(dev))
    rh, ri = layer.experts_mod.rot_h, layer.experts_mod.rot_i
    ref = O.moe_layer(h, logits, cb, gu, gus, dn, dns, gu[E], gus[E], dn[E], dns[E], gate,
                      rh.perm.cpu().numpy(), rh.sign.float().cpu().numpy(), ri.perm.cpu().numpy(),
                      ri.sign.float().cpu().numpy(), top_k=k)
    assert out.shape == (T, 2048)
    assert O.max_rel_err(out.cpu().numpy(), ref) < TOL


def test_resident_experts_drop_in_forward(dev):
    """PackedMoEExpertUniversal.forward(hidden, topk_idx, topk_weights) shape."""
    from compressai_amd.moe import ResidentMoEExperts

    E = 16
    cb = synth.codebook(4400)
    gu, gus, dn, dns = _pools(4400, E)
    mod = ResidentMoEExperts.from_pools(*_cuda(gu, gus, dn, dns, cb, dev=dev))
    h = synth.activations(4404, (2, 2048), dtype=torch.bfloat16)
    ids = torch.tensor([[1, 4, 9, 15, 0, 2, 3, 8], [15, 14, 1, 0, 5, 6, 7, 4]], dtype=torch.int64)
    w = torch.softmax(synth.activations(4405, (2, 8)).float(), -1).to(torch.bfloat16)
    out = mod(h.to(dev), ids.to(dev), w.to(dev))
    assert out.shape == (2, 2048) and out.dtype == torch.bfloat16
    rh, ri = mod.rot_h, mod.rot_i
    ref = np.zeros((2, 2048))
    for t in range(2):
        xr = O.np_rht64(h[t], rh.perm.cpu().numpy(), rh.sign.float().cpu().numpy(), 2048)[0]
        for j in range(8):
            e = int(ids[t, j])
            Wgu = O.np_dequant64(gu[e], None, cb, None, gus[e])
            g = Wgu @ xr
            act = O.silu(g[:512]) * g[512:]
            ar = O.np_rht64(act, ri.perm.cpu().numpy(), ri.sign.float().cpu().numpy(), 512)[0]
            ref[t] += float(w[t, j]) * (O.np_dequant64(dn[e], None, cb, None, dns[e]) @ ar)
    assert O.max_rel_err(out.float().cpu().numpy(), ref) < 8e-3  # bf16 output rounding


# ------------------------------------------------------- fused-RHT launches
@pytest.mark.parametrize("bpw", [2, 3, 4])
@pytest.mark.parametrize("batch", [1, 2])
def test_gemv_rht_fused_segments(dev, bpw, batch):
    """RHT + q/k/v-style multi-matrix GEMV in one launch vs RHT then GEMV."""
    n = 2048
    cb0 = synth.codebook(9100)
    cb1 = synth.codebook(9101, 256 if bpw == 3 else 65536) if bpw > 2 else None
    shapes = [2048, 512, 512]
    mats = [synth.vq_matrix(9100 + 10 * k, rows, n, bpw=bpw) for k, rows in enumerate(shapes)]
    x = synth.activations(9104, (batch, n), dtype=torch.float16)
    perm = synth.permutation(9106, n)
    sign = synth.signs(9105, n)
    ys = K.vq_gemv_rht(x.to(dev), [(m["idx0"].to(dev), None if m["idx1"] is None else m["idx1"].to(dev),
                                    m["scale"].to(dev), rows) for m, rows in zip(mats, shapes)],
                       cb0.to(dev), None if cb1 is None else cb1.to(dev), n, perm.to(dev), sign.to(dev), 2048)
    xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    for y, m, rows in zip(ys, mats, shapes):
        _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
        assert y.shape == (batch, rows)
        assert O.max_rel_err(y.cpu().numpy(), y64) < TOL


@pytest.mark.parametrize("hb", [2, 8, 16, 32, 64, 512])
@pytest.mark.parametrize("batch", [1, 2])
def test_gemv_rht_fused_small_blocks(dev, hb, batch):
    """Fused RHT with blocks shorter than the in-register / cross-lane FWHT
    stages (hb < 64 stops inside them) against RHT then GEMV."""
    n, out = 512, 700
    cb0 = synth.codebook(9150)
    m = synth.vq_matrix(9150 + hb, out, n, bpw=2)
    x = synth.activations(9154 + hb, (batch, n), dtype=torch.float16)
    perm = synth.permutation(9156, n)
    sign = synth.signs(9155, n)
    (y,) = K.vq_gemv_rht(x.to(dev), [(m["idx0"].to(dev), None, m["scale"].to(dev), out)], cb0.to(dev), None, n,
                         perm.to(dev), sign.to(dev), hb)
    xr = O.rht(x, perm, sign, hb).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], None, cb0, None, m["scale"])
    assert O.max_rel_err(y.cpu().numpy(), y64) < TOL


def test_gemv_rht_fused_6144(dev):
    """down projection: 2048 x 6144 at 4 bpw with its 3 x 2048-block RHT fused."""
    n, out = 6144, 2048
    cb0, cb1 = synth.codebook(9200), synth.codebook(9201)
    m = synth.vq_matrix(9200, out, n, bpw=4)
    x = synth.activations(9204, n, dtype=torch.float16)
    sign = synth.signs(9205, n)
    (y,) = K.vq_gemv_rht(x.to(dev), [(m["idx0"].to(dev), m["idx1"].to(dev), m["scale"].to(dev), out)],
                         cb0.to(dev), cb1.to(dev), n, None, sign.to(dev), 2048)
    xr = O.rht(x, None, sign, 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL


@pytest.mark.parametrize("n,batch,bpw,xdt", [
    (6144, 1, 4, torch.float16), (6144, 1, 2, torch.float32), (6144, 1, 3, torch.bfloat16),
    (4096, 1, 4, torch.float32), (3072, 2, 2, torch.float16), (2048, 2, 3, torch.bfloat16)])
def test_gemv_rht_fused_wide(dev, n, batch, bpw, xdt):
    """Activation blocks wider than 256 threads x 8 values rotate in one pass
    of a wider workgroup (up to 768 threads): permuted RHT + GEMV against the
    oracle's RHT then GEMV, every codebook stage kind and activation dtype."""
    out = 1000
    cb0 = synth.codebook(9400)
    cb1 = synth.codebook(9401, 256 if bpw == 3 else 65536) if bpw > 2 else None
    m = synth.vq_matrix(9400 + n + batch, out, n, bpw=bpw)
    x = synth.activations(9404 + n, (batch, n), dtype=xdt)
    perm = synth.permutation(9406 + n, n)
    sign = synth.signs(9405 + n, n)
    hb = 2048 if n % 2048 == 0 else 1024
    (y,) = K.vq_gemv_rht(x.to(dev), [(m["idx0"].to(dev), None if m["idx1"] is None else m["idx1"].to(dev),
                                      m["scale"].to(dev), out)], cb0.to(dev), None if cb1 is None else cb1.to(dev),
                         n, perm.to(dev), sign.to(dev), hb)
    xr = O.rht(x.float(), perm, sign, hb).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert y.shape == (batch, out)
    assert O.max_rel_err(y.cpu().numpy(), y64) < TOL


@pytest.mark.parametrize("n,batch", [(2048, 1), (2048, 2), (6144, 1)])
@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_gemv_rht_fused_unaligned_activation(dev, n, batch, xdt):
    """The fused prologue's activation loads (8 contiguous elements per
    thread) from rows that start one element past 16-byte alignment."""
    out, bpw = 700, 2
    cb0 = synth.codebook(9450)
    m = synth.vq_matrix(9450 + n + batch, out, n, bpw=bpw)
    flat = synth.activations(9454 + n, batch * n + 8, dtype=xdt)
    xh = flat[1:1 + batch * n].view(batch, n)
    x = flat.to(dev)[1:1 + batch * n].view(batch, n)  # contiguous, storage offset 1
    perm = synth.permutation(9456 + n, n)
    sign = synth.signs(9455 + n, n)
    (y,) = K.vq_gemv_rht(x, [(m["idx0"].to(dev), None, m["scale"].to(dev), out)], cb0.to(dev), None, n,
                         perm.to(dev), sign.to(dev), 2048)
    xr = O.rht(xh.float(), perm, sign, 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], None, cb0, None, m["scale"])
    assert O.max_rel_err(y.cpu().numpy(), y64) < TOL


@pytest.mark.parametrize("n,batch", [(2048, 2), (6144, 1)])
def test_gemv_rht_fused_bad_perm_entry_poisons(dev, n, batch):
    """An out-of-range permutation entry in the fused prologue (staged in
    LDS) reads in bounds and poisons its batch row: every output of that row
    is NaN; with a valid permutation the same launch matches the oracle."""
    out = 600
    cb0 = synth.codebook(9470)
    m = synth.vq_matrix(9470 + n, out, n, bpw=2)
    x = synth.activations(9474 + n, (batch, n), dtype=torch.float16)
    perm = synth.permutation(9476 + n, n)
    sign = synth.signs(9475 + n, n)
    pbad = perm.clone()
    pbad[n // 3] = -7
    mats = [(m["idx0"].to(dev), None, m["scale"].to(dev), out)]
    (y,) = K.vq_gemv_rht(x.to(dev), mats, cb0.to(dev), None, n, pbad.to(dev), sign.to(dev), 2048)
    assert torch.isnan(y).all()
    (y2,) = K.vq_gemv_rht(x.to(dev), mats, cb0.to(dev), None, n, perm.to(dev), sign.to(dev), 2048)
    xr = O.rht(x.float(), perm, sign, 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], None, cb0, None, m["scale"])
    assert O.max_rel_err(y2.cpu().numpy(), y64) < TOL


def test_gemv_empty_segments(dev):
    """Zero-row matrices: a launch with no rows is a no-op, and an empty
    segment between non-empty ones (whose row blocks it owns none of) does not
    shift the others' rows."""
    n = 2048
    cb0 = synth.codebook(9500)
    m = synth.vq_matrix(9500, 0, n, bpw=2)
    y = K.vq_gemv_16(synth.activations(9504, n, dtype=torch.float32).to(dev), m["idx0"].to(dev), cb0.to(dev),
                     m["scale"].to(dev), 0, n, 1.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert y.shape == (0,)
    shapes = [512, 0, 300, 0]
    mats = [synth.vq_matrix(9510 + 10 * k, rows, n, bpw=2) for k, rows in enumerate(shapes)]
    x = synth.activations(9514, n, dtype=torch.float16)
    sign = synth.signs(9515, n)
    ys = K.vq_gemv_rht(x.to(dev), [(mm["idx0"].to(dev), None, mm["scale"].to(dev), rows) for mm, rows in zip(mats, shapes)],
                       cb0.to(dev), None, n, None, sign.to(dev), 2048)
    xr = O.rht(x, None, sign, 2048).astype(np.float32)
    for yk, mm, rows in zip(ys, mats, shapes):
        assert yk.shape == (rows,)
        if rows:
            _, y64 = O.vq_gemv(xr, mm["idx0"], None, cb0, None, mm["scale"])
            assert O.max_rel_err(yk.cpu().numpy(), y64[0]) < TOL


def test_packed_linear_forward(dev):
    from compressai_amd.runtime import PackedLinear, PackedLMHead

    n, out = 2048, 1536
    cbs = {"16": synth.codebook(9300).to(dev), "16_16": synth.codebook(9301).to(dev)}
    m = synth.vq_matrix(9300, out, n, bpw=4)
    lin = PackedLinear((out, n), (16, 16), "layers.0.mlp.gate_proj", [m["idx0"], m["idx1"]], m["scale"], cbs, dev)
    for B in (1, 3):  # fused single launch (B <= 2) and the two-launch path
        x = synth.activations(9304 + B, (B, n), dtype=torch.float32)
        y = lin(x.to(dev))
        xr = O.rht(x, lin.rot.perm.cpu(), lin.rot.sign.float().cpu().numpy().astype(np.int8), lin.rot.hb)
        _, y64 = O.vq_gemv(xr.astype(np.float32), m["idx0"], m["idx1"], cbs["16"], cbs["16_16"], lin.scale.cpu())
        assert O.max_rel_err(y.cpu().numpy(), y64) < TOL
    head = PackedLMHead(lin)
    idx, val = head.argmax(synth.activations(9310, (2, n), dtype=torch.float32).to(dev))
    logits = head(synth.activations(9310, (2, n), dtype=torch.float32).to(dev))
    assert idx.cpu().tolist() == logits.argmax(-1).cpu().tolist()


@pytest.mark.parametrize("T", [1, 3])
def test_moe_fused_launches_vs_unfused(dev, T):
    """gate_up+RHT and SwiGLU+RHT+down+combine launches vs the separate kernels."""
    E, P = 12, 5
    cb = synth.codebook(9400).to(dev)
    gu, gus, dn, dns = (t.to(dev) for t in _pools(9400, E))
    ids = torch.randint(0, E, (T, P), generator=synth.gen(9401), dtype=torch.int32).to(dev)
    w = torch.rand(T, P, generator=synth.gen(9402)).to(dev)
    h = synth.activations(9403, (T, 2048), dtype=torch.float16).to(dev)
    sign_h, sign_i = synth.signs(9404, 2048).to(dev), synth.signs(9405, 512).to(dev)
    perm_h, perm_i = synth.permutation(9406, 2048).to(dev), synth.permutation(9407, 512).to(dev)
    y_gu = torch.empty(T * P, 1024, device=dev)
    K.vq_moe_gate_up_rht(h, ids, gu, cb, gus, y_gu, 1024, 256, perm_h, sign_h, 2048)
    xr = K.vq_rht(h, perm_h, sign_h, 2048, out_dtype=torch.float32)
    ref_gu = torch.empty(T * P, 1024, device=dev)
    K.vq_moe_grouped(xr, ids, gu, cb, gus, ref_gu, 1024, 256, pairs_per_x=P)
    assert O.max_rel_err(y_gu.cpu().numpy(), ref_gu.double().cpu().numpy()) < 1e-5
    out = K.vq_moe_down_swiglu_combine(y_gu, ids, w, dn, cb, dns, 2048, 64, perm_i, sign_i, 512)
    act_r = K.vq_swiglu_rht(y_gu, 512, perm_i, sign_i, 512)
    ref = K.vq_moe_down_combine(act_r, ids, w, dn, cb, dns, OUT=2048, NG=64)
    assert O.max_rel_err(out.cpu().numpy(), ref.double().cpu().numpy()) < 1e-5


# ----------------------------------------------------- small-M MFMA GEMM
def _rowwise_err(y, ref):
    return max(O.max_rel_err(y[b], ref[b]) for b in range(ref.shape[0]))


@pytest.mark.parametrize("out,n,bpw", [(6144, 2048, 2), (2048, 6144, 4), (1000, 512, 3), (517, 2048, 4)])
@pytest.mark.parametrize("M", [2, 5, 16, 17, 64])
def test_gemm_small_m_vs_oracle(dev, out, n, bpw, M):
    """Every batch row within 1e-3 of the fp64 oracle (x and centroids go
    through fp16 with a per-row power-of-two scale)."""
    m = synth.vq_matrix(7000 + out + bpw, out, n, bpw=bpw)
    cb0 = synth.codebook(7001)
    cb1 = synth.codebook(7002, 256 if bpw == 3 else 65536) if bpw > 2 else None
    x = synth.activations(7004 + M, (M, n), dtype=torch.float32)
    i0, i1, sc, c0, c1, xx = _cuda(m["idx0"], m["idx1"], m["scale"], cb0, cb1, x, dev=dev)
    y = K.vq_gemm_small_m(xx, i0, i1, c0, c1, sc, out, n, 0.5, out_dtype=torch.float32)
    _, y64 = O.vq_gemv(x, m["idx0"], m["idx1"], cb0, cb1, m["scale"], 0.5)
    assert y.shape == (M, out)
    assert _rowwise_err(y.cpu().numpy(), y64) < TOL


@pytest.mark.parametrize("cbdt,xdt,ydt", [(torch.bfloat16, torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.float16, torch.float32),
                                          (torch.float16, torch.bfloat16, torch.float16)])
def test_gemm_small_m_dtypes(dev, cbdt, xdt, ydt):
    out, n, M = 768, 2048, 24
    m = synth.vq_matrix(7100, out, n, bpw=4)
    cb0 = synth.codebook(7101, dtype=cbdt)
    cb1 = synth.codebook(7102, dtype=cbdt)
    x = synth.activations(7104, (M, n), dtype=xdt)
    sc = m["scale"].to(torch.bfloat16) if cbdt == torch.bfloat16 else m["scale"]
    i0, i1, s_, c0, c1, xx = _cuda(m["idx0"], m["idx1"], sc, cb0, cb1, x, dev=dev)
    y = K.vq_gemm_small_m(xx, i0, i1, c0, c1, s_, out, n, out_dtype=ydt)
    _, y64 = O.vq_gemv(x, m["idx0"], m["idx1"], cb0, cb1, sc)
    tol = TOL if ydt == torch.float32 else 2.0 ** -8 + TOL
    assert y.dtype == ydt and _rowwise_err(y.float().cpu().numpy(), y64) < tol


def test_gemm_small_m_extreme_rows(dev):
    """Rows scaled by 1e6 and 1e-6 (fp16 alone would overflow / lose them),
    a zero row, and a NaN row that stays confined to its own outputs."""
    out, n, M = 640, 1024, 6
    m = synth.vq_matrix(7200, out, n, bpw=2)
    cb0 = synth.codebook(7201)
    x = synth.activations(7204, (M, n), dtype=torch.float32)
    x[1] *= 1e6
    x[2] *= 1e-6
    x[3] = 0.0
    x[4, 17] = float("nan")
    i0, sc, c0, xx = _cuda(m["idx0"], m["scale"], cb0, x, dev=dev)
    y = K.vq_gemm_small_m(xx, i0, None, c0, None, sc, out, n, out_dtype=torch.float32).cpu().numpy()
    xo = x.clone()
    xo[4] = 0.0
    _, y64 = O.vq_gemv(xo, m["idx0"], None, cb0, None, m["scale"])
    for b in (0, 1, 2, 5):
        assert O.max_rel_err(y[b], y64[b]) < TOL, b
    assert np.all(y[3] == 0.0)
    assert np.all(np.isnan(y[4]))


def test_gemm_small_m_matches_batched_gemv(dev):
    """Same inputs through vq2_gemm_small_m and the batched vq2_gemv: the two
    kernels agree to the output tolerance, on two calls in a row with the
    second one smaller (the shared split-K workspace is reused)."""
    for out, M in [(6144, 64), (2048, 16)]:
        m = synth.vq_matrix(7300 + M, out, 2048, bpw=2)
        cb0 = synth.codebook(7301)
        x = synth.activations(7304 + M, (M, 2048), dtype=torch.float16)
        i0, sc, c0, xx = _cuda(m["idx0"], m["scale"], cb0, x, dev=dev)
        ya = K.vq_gemm_small_m(xx, i0, None, c0, None, sc, out, 2048, out_dtype=torch.float32)
        yb = K.vq_gemv(xx, i0, None, c0, None, sc, out, 2048, out_dtype=torch.float32)
        assert _rowwise_err(ya.cpu().numpy(), yb.cpu().numpy()) < TOL


def test_gemm_small_m_split_sum_in_launch_is_deterministic(dev):
    """The K splits are summed inside the launch by the last workgroup of
    each row tile to arrive (arrival counters in the workspace header): the
    same result on every call, interleaved with sorted launches that share
    the workspace, and on every replay of a captured graph (with eager work
    between the replays), bit for bit; and the counters are left at zero."""
    out, n, M = 6144, 2048, 64
    m = synth.vq_matrix(7350, out, n, bpw=4)
    cb0, cb1 = synth.codebook(7351), synth.codebook(7352)
    x = synth.activations(7354, (M, n), dtype=torch.float16)
    i0, i1, sc, c0, c1, xx = _cuda(m["idx0"], m["idx1"], m["scale"], cb0, cb1, x, dev=dev)
    y0 = K.vq_gemm_small_m(xx, i0, i1, c0, c1, sc, out, n, out_dtype=torch.float32)
    _, y64 = O.vq_gemv(x, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert _rowwise_err(y0.cpu().numpy(), y64) < TOL
    sp = K.SortedPlanes(m["idx0"], m["idx1"], out, n, device=dev)
    ys = K.vq_sorted_gemv(xx[0], [(sp, sc)], c0, c1, n, hb=0)
    y1 = K.vq_gemm_small_m(xx, i0, i1, c0, c1, sc, out, n, out_dtype=torch.float32)
    assert torch.equal(y0, y1)
    y = torch.empty_like(y0)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        K.vq_gemm_small_m(xx, i0, i1, c0, c1, sc, out, n, out_dtype=torch.float32, y=y)
    torch.cuda.current_stream(dev).wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.vq_gemm_small_m(xx, i0, i1, c0, c1, sc, out, n, out_dtype=torch.float32, y=y)
    for _ in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(y, y0)
        K.vq_sorted_gemv(xx[1], [(sp, sc)], c0, c1, n, hb=0, ys=ys)
    torch.cuda.synchronize(dev)
    for ws in [t for k, t in K._WS.items() if k[0] == dev.index and k[2]]:
        assert int(ws[:K.WS_STATUS].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("B", [3, 70])
def test_packed_linear_small_m_path(dev, B):
    """PackedLinear at batch >= 3 (matrix-core GEMM, chunked at 64 rows)
    against the fp64 oracle of RHT + VQ GEMV."""
    from compressai_amd.runtime import PackedLinear
    out, n = 512, 2048
    m = synth.vq_matrix(7400, out, n, bpw=4)
    cbs = {"16": synth.codebook(7401).to(dev), "16_16": synth.codebook(7402).to(dev)}
    lin = PackedLinear((out, n), (16, 16), "t_small_m", [m["idx0"], m["idx1"]], m["scale"], cbs, dev)
    x = synth.activations(7404, (B, n), dtype=torch.float32)
    y = lin(x.to(dev), out_dtype=torch.float32).cpu().numpy()
    xr = O.rht(x, lin.rot.perm.cpu(), lin.rot.sign.float().cpu().numpy().astype(np.int8), lin.rot.hb)
    _, y64 = O.vq_gemv(xr.astype(np.float32), m["idx0"], m["idx1"], cbs["16"].cpu(), cbs["16_16"].cpu(),
                       lin.scale.cpu())
    assert y.shape == (B, out)
    assert _rowwise_err(y, y64) < TOL


def test_lm_head_argmax_small_m_batch(dev):
    """vq_gemv_argmax at batch 5 (matrix-core path) picks the oracle's top-1."""
    out, n, B = 4096, 2048, 5
    m = synth.vq_matrix(7500, out, n, bpw=2)
    cb = synth.codebook(7501)
    x = synth.activations(7504, (B, n), dtype=torch.float32)
    idx, val = K.vq_gemv_argmax(x.to(dev), m["idx0"].to(dev), None, cb.to(dev), None, m["scale"].to(dev), out, n)
    _, y64 = O.vq_gemv(x, m["idx0"], None, cb, None, m["scale"])
    ref = O.argmax_rows(y64)
    # a different top-1 is only acceptable within the output tolerance of a tie
    for b in range(B):
        if int(idx[b]) != int(ref[b]):
            assert abs(y64[b, int(idx[b])] - y64[b, int(ref[b])]) <= TOL * np.abs(y64[b]).max()


@pytest.mark.parametrize("B,out,bpw", [(3, 4096, 2), (4, 40000, 2), (17, 3000, 4), (64, 2048, 3), (70, 1000, 2)])
def test_small_m_fused_top1_equals_logits_argmax(dev, B, out, bpw):
    """The matrix-core LM-head top-1 (top-1 fused into the split-K reduce, no
    logits written) returns exactly torch.argmax / the value of the same
    GEMM's fp32 logits, including a tie placed across reduce blocks."""
    n = 2048
    m = synth.vq_matrix(7600 + B, out, n, bpw=bpw)
    cbs = {2: (synth.codebook(7601), None), 3: (synth.codebook(7601), synth.codebook(7602, rows=256)),
           4: (synth.codebook(7601), synth.codebook(7603))}[bpw]
    i1 = m.get("idx1")
    i0 = m["idx0"].clone()
    sc = m["scale"].clone()
    if out > 600:  # rows 300 and out-1 identical and scaled up: a tie that wins where its dot is > 0
        i0[out - 1] = i0[300]
        sc[300] = sc[out - 1] = 12.0
        if i1 is not None:
            i1 = i1.clone()
            i1[out - 1] = i1[300]
    x = synth.activations(7604 + B, (B, n), dtype=torch.float32)
    args = _cuda(x, i0, i1, cbs[0], cbs[1], sc, dev=dev)
    idx, val = K.vq_gemv_argmax(*args, out, n)
    logits = torch.cat([K.vq_gemm_small_m(args[0][b0:b0 + 64], *args[1:], out, n, out_dtype=torch.float32)
                        for b0 in range(0, B, 64)])
    ref_val, ref_idx = torch.max(logits, dim=1)
    assert torch.equal(idx, torch.argmax(logits, dim=1))
    assert torch.equal(val, ref_val)
    if out > 600:
        assert torch.equal(logits[:, 300], logits[:, out - 1])
        assert not torch.any(idx == out - 1)  # the first of the tied rows
        assert torch.any(idx == 300)


@pytest.mark.parametrize("E,k,shared,T", [(256, 8, True, 1), (256, 8, True, 8), (300, 4, False, 3),
                                          (64, 2, True, 5)])
def test_fused_router_gate_up_matches_router_and_unfused(dev, E, k, shared, T):
    """vq2_moe_router_gate_up_rht: ids and weights bit-identical to the
    standalone router (E > 256 takes the 16-logits-per-lane path), gate_up
    rows identical to vq2_moe_gate_up_rht fed those ids."""
    NG, OUT = 32, 128  # n = 256 (hb 256), 2I = 128
    g = torch.Generator().manual_seed(4500 + E + T)
    pool = torch.randint(-32768, 32768, (E + 1, OUT, NG), generator=g, dtype=torch.int32).to(torch.int16)
    ps = (torch.rand(E + 1, OUT, generator=g) + 0.5).to(torch.float16)
    cb = synth.codebook(4501)
    h = synth.activations(4504 + T, (T, NG * 8))
    logits = synth.activations(4507 + T, (T, E))
    gate = synth.activations(4508, NG * 8) * 0.05
    sign = synth.signs(4509, NG * 8)
    sid = E if shared else -1
    P = k + (1 if shared else 0)
    pool_d, ps_d, cb_d, h_d, lg_d, gate_d, sign_d = _cuda(pool, ps, cb, h, logits, gate, sign, dev=dev)
    y1 = torch.empty((T * P, OUT), dtype=torch.float32, device=dev)
    ids, w = K.vq_moe_router_gate_up_rht(h_d, lg_d, k, pool_d, cb_d, ps_d, y1, OUT, NG, shared_gate=gate_d,
                                         shared_id=sid, sign=sign_d, hb=256)
    rid, rw = K.vq_router_topk(lg_d, k, h_d if shared else None, gate_d if shared else None, shared_id=sid)
    assert torch.equal(ids.cpu(), rid.cpu().to(torch.int32))
    assert torch.equal(w.cpu(), rw.cpu())
    y2 = torch.empty_like(y1)
    K.vq_moe_gate_up_rht(h_d, rid, pool_d, cb_d, ps_d, y2, OUT, NG, sign=sign_d, hb=256)
    assert torch.equal(y1.cpu(), y2.cpu())


# ------------------------------------------------------------ unpack_fixed
from vq2_containers import pack_fixed as _pack  # noqa: E402


@pytest.mark.parametrize("bits", [4, 8, 12, 16])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 100003])
def test_unpack_fixed_round_trip(dev, bits, n):
    rng = np.random.default_rng(bits * 1000 + n)
    sym = rng.integers(0, 1 << bits, n, dtype=np.int64)
    buf = _pack(sym, bits)
    got = K.vq_unpack_fixed(torch.from_numpy(buf).to(dev), bits, n).cpu().numpy().view(np.uint16)
    assert np.array_equal(got.astype(np.int64), sym)
    assert np.array_equal(got.astype(np.int64), O.unpack_fixed(buf, bits, n))


def test_unpack_fixed_misaligned_and_short(dev):
    """A stream that starts at an odd byte takes the per-symbol path; a
    buffer shorter than ceil(n * bits / 8) is refused."""
    sym = np.random.default_rng(5).integers(0, 4096, 333, dtype=np.int64)
    buf = np.concatenate([np.zeros(1, np.uint8), _pack(sym, 12)])
    t = torch.from_numpy(buf).to(dev)
    got = K.vq_unpack_fixed(t[1:], 12, 333).cpu().numpy().view(np.uint16)
    assert np.array_equal(got.astype(np.int64), sym)
    with pytest.raises(K.Vq2Error):
        K.vq_unpack_fixed(t[1:-2], 12, 333)


# ------------------------------------------------------- paged expert pool
def test_paged_experts_match_resident_pool(dev, tmp_path):
    """PagedMoEExperts (container -> pinned ring -> slot pool, LRU with
    evictions) gives the resident pool's outputs over a sequence of steps."""
    from compressai_amd import paged
    from compressai_amd.moe import ResidentMoEExperts
    E = 16
    g = torch.Generator().manual_seed(4600)
    gui = torch.randint(-32768, 32768, (E, 1024, 256), generator=g, dtype=torch.int32).to(torch.int16)
    gus = (torch.rand(E, 1024, generator=g) + 0.5).to(torch.float16)
    dni = torch.randint(-32768, 32768, (E, 2048, 64), generator=g, dtype=torch.int32).to(torch.int16)
    dns = (torch.rand(E, 2048, generator=g) + 0.5).to(torch.float16)
    path = tmp_path / "moe.vq2m"
    paged.write_vq2m(path, [gui], [gus], [dni], [dns])
    cb = synth.codebook(4601).to(dev)
    store = paged.Vq2mStore(path)
    pg = paged.PagedMoEExperts(0, store, cb, capacity=6, device=dev, staging=3, out_dtype=torch.float32)
    # the paged pool holds bf16-rounded scales (as the reference's pools): same for the resident one
    bf = torch.bfloat16
    # (the gather kernels on the reference pools, which the paged feed runs too)
    res = ResidentMoEExperts.from_pools(gui.to(dev), gus.to(dev, bf), dni.to(dev), dns.to(dev, bf), cb,
                                        out_dtype=torch.float32, sorted_layout=False)
    for step in range(8):
        T = 1 + step % 3
        ids = torch.stack([torch.randperm(E, generator=g)[:2] for _ in range(T)]).to(torch.int64)
        w = torch.softmax(torch.randn(T, 2, generator=g), -1)
        h = synth.activations(4610 + step, (T, 2048), dtype=torch.float16)
        yp = pg(h.to(dev), ids.to(dev), w.to(dev))
        yr = res(h.to(dev), ids.to(dev), w.to(dev))
        assert torch.equal(yp.cpu(), yr.cpu()), step
    assert pg.pager.misses > 6 and pg.pager.hits > 0  # evictions happened and some experts stayed
    store.close()


def _rot_np(rot):
    return rot.perm.cpu().numpy(), rot.sign.float().cpu().numpy()


@pytest.mark.parametrize("T", [1, 3])
def test_single_pair_combine_applies_weight(dev, T):
    """One expert per token (P = 1): both combines scale by the pair weight
    (a single-pair workgroup still runs the weighted store)."""
    from compressai_amd.moe import ResidentMoEExperts

    E = 6
    cb = synth.codebook(4900)
    gu, gus, dn, dns = _pools(4900, E)
    mod = ResidentMoEExperts.from_pools(*_cuda(gu, gus, dn, dns, cb, dev=dev), out_dtype=torch.float32)
    h = synth.activations(4904, (T, 2048))
    ids = torch.tensor([[2], [5], [0]][:T], dtype=torch.int32)
    w = torch.tensor([[0.37], [-1.5], [2.25]][:T], dtype=torch.float32)
    out = mod(h.to(dev), ids.to(dev), w.to(dev))
    ph, sh = _rot_np(mod.rot_h)
    pi, si = _rot_np(mod.rot_i)
    ref = O.moe_experts(h, ids.numpy(), w.numpy(), lambda e: (gu[e], None, gus[e], dn[e], None, dns[e]), cb,
                        None, ph, sh, pi, si)
    assert O.max_rel_err(out.cpu().numpy(), ref) < TOL
    # the split down + combine launch as well
    act = synth.activations(4905, (T, 512), dtype=torch.float32)
    y = K.vq_moe_down_combine(act.to(dev), ids.to(dev), w.to(dev), *_cuda(dn, cb, dns, dev=dev), OUT=2048, NG=64)
    ref2 = np.stack([float(w[t, 0]) * O.vq_gemv(act[t], dn[int(ids[t, 0])], None, cb, None,
                                                  dns[int(ids[t, 0])])[1][0] for t in range(T)])
    assert O.max_rel_err(y.cpu().numpy(), ref2) < TOL


def test_paged_promoted_experts_vs_oracle(dev, tmp_path):
    """A layer with promoted (16,8) experts: steps with mixed, only-promoted
    and only-2-bpw tokens, the 2 bpw pairs through the two fused launches on
    the paged pool and the promoted pairs through the one-launch sorted MoE
    on the two-stage sorted pool (added to the 2 bpw sum), against the fp64
    oracle."""
    from compressai_amd import paged

    E = 12
    pro = (3, 7, 10)
    g = torch.Generator().manual_seed(4950)
    gui = torch.randint(-32768, 32768, (E, 1024, 256), generator=g, dtype=torch.int32).to(torch.int16)
    gus = (torch.rand(E, 1024, generator=g) + 0.5).to(torch.float16)
    dni = torch.randint(-32768, 32768, (E, 2048, 64), generator=g, dtype=torch.int32).to(torch.int16)
    dns = (torch.rand(E, 2048, generator=g) + 0.5).to(torch.float16)
    gu1 = torch.randint(0, 256, (E, 1024, 256), generator=g, dtype=torch.int32).to(torch.uint8)
    dn1 = torch.randint(0, 256, (E, 2048, 64), generator=g, dtype=torch.int32).to(torch.uint8)
    path = tmp_path / "mixed.vq2m"
    paged.write_vq2m(path, [gui], [gus], [dni], [dns], promoted={(0, e): (gu1[e], dn1[e]) for e in pro})
    cb = synth.codebook(4951)
    cb8 = synth.codebook(4952, rows=256)
    store = paged.Vq2mStore(path)
    pg = paged.PagedMoEExperts(0, store, cb.to(dev), capacity=4, device=dev, staging=2, out_dtype=torch.float32,
                               cb8=cb8.to(dev))
    assert pg.pro_sorted is not None and pg.pro_sorted[0].s2_kind == 2  # promoted pairs on the sorted path
    ph, sh = _rot_np(pg.rot_h)
    pi, si = _rot_np(pg.rot_i)

    def experts(e):  # the pools hold bf16-rounded scales, as the reference's
        p = e in pro
        bf = torch.bfloat16
        return gui[e], gu1[e] if p else None, gus[e].to(bf), dni[e], dn1[e] if p else None, dns[e].to(bf)

    steps = [[[3, 5]], [[3, 7], [1, 2], [10, 4]], [[7, 10], [3, 7]], [[3, 5, 6]], [[5, 6], [0, 1]], [[10, 0]]]
    for i, rows in enumerate(steps):
        ids = torch.tensor(rows, dtype=torch.int64)
        T, P = ids.shape
        w = torch.softmax(torch.randn(T, P, generator=g), -1)
        h = synth.activations(4960 + i, (T, 2048), dtype=torch.float16)
        y = pg(h.to(dev), ids.to(dev), w.to(dev))
        ref = O.moe_experts(h, ids.numpy(), w.numpy(), experts, cb, cb8, ph, sh, pi, si)
        assert O.max_rel_err(y.cpu().numpy(), ref) < TOL, (i, rows)
    store.close()


# ------------------------------------------------------------ graph capture
def test_decode_step_graph_replays_match_eager(dev):
    """One decode step -- fused q/k/v (PackedLinear, batch 1), a 4 bpw
    projection, the MoE layer (router inside gate_up) and the LM-head top-1 --
    captured once; every replay, with eager work and synchronisations between
    replays, equals the eager step on the same input."""
    from compressai_amd.graph import DecodeStepGraph
    from compressai_amd.moe import MoELayer
    from compressai_amd.runtime import PackedLinear

    n = 2048
    cbs = {"16": synth.codebook(4700).to(dev), "16_16": synth.codebook(4701).to(dev)}
    mq = synth.vq_matrix(4700, 1024, n, bpw=2)
    mg = synth.vq_matrix(4710, 768, n, bpw=4)
    lin_q = PackedLinear((1024, n), (16,), "layers.0.self_attn.q_proj", [mq["idx0"]], mq["scale"], cbs, dev)
    lin_g = PackedLinear((768, n), (16, 16), "layers.0.mlp.gate_proj", [mg["idx0"], mg["idx1"]], mg["scale"], cbs,
                         dev)
    E, k = 32, 4
    gu, gus, dn, dns = _pools(4720, E + 1)
    moe = MoELayer(*_cuda(gu, gus, dn, dns, cbs["16"], synth.activations(4721, n) * 0.02, dev=dev), top_k=k)
    head_m = synth.vq_matrix(4730, 4096, n, bpw=2)
    head = PackedLinear((4096, n), (16,), "lm_head", [head_m["idx0"]], head_m["scale"], cbs, dev)

    def step(x, logits):
        q = lin_q(x, out_dtype=torch.float32)
        gt = lin_g(x, out_dtype=torch.float32)
        y = moe(x, logits)
        xr = head.rot.fwd(x.reshape(1, n), out_dtype=torch.float32)
        i0, _, cb0, _ = head._planes()
        idx, val = K.vq_gemv_argmax(xr, i0, None, cb0, None, head.scale, 4096, n)
        return q, gt, y, idx, val

    x0 = synth.activations(4740, (1, n)).to(dev)
    l0 = synth.activations(4741, (1, E)).to(dev)
    gstep = DecodeStepGraph(step, [x0, l0])
    for r in range(4):
        x = synth.activations(4750 + r, (1, n)).to(dev)
        lg = synth.activations(4760 + r, (1, E)).to(dev)
        ref = [t.clone() for t in step(x, lg)]
        torch.cuda.synchronize()
        out = [t.clone() for t in gstep(x, lg)]
        torch.cuda.synchronize()
        for a, b in zip(out, ref):
            assert torch.equal(a, b), r


@pytest.mark.parametrize("B,n", [(1, 2048), (2, 2048), (1, 4096)])
def test_fused_top1_ties_and_fallback(dev, B, n):
    """Rows 700 and 3000 are identical and hold the maximum of every batch
    column: the fused top-1 (n = 2048) and the logits + top-1 fallback
    (n = 4096, two K chunks) both return the lower row, as torch.argmax."""
    out = 4096
    m = synth.vq_matrix(4800 + n, out, n, bpw=2)
    i0 = m["idx0"].clone()
    i0[3000] = i0[700]
    sc = m["scale"].clone()
    cb = synth.codebook(4801)
    x = synth.activations(4802 + B, (B, n), dtype=torch.float32)
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    sign = np.sign(y64[:, 700])  # make the tied pair the maximum of each column
    x = x * torch.from_numpy(sign.astype(np.float32))[:, None]
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    unit = y64[:, 700] / float(sc[700])
    need = np.abs(y64).max() / unit.min()
    sc[700] = sc[3000] = float(2.0 ** np.ceil(np.log2(need) + 1))
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    assert np.all(np.argmax(y64, 1) == 700) and np.all(y64[:, 700] == y64[:, 3000])
    idx, val = K.vq_gemv_argmax(*_cuda(x, i0, None, cb, None, sc, dev=dev), out, n)
    assert idx.cpu().tolist() == [700] * B
    assert np.allclose(val.cpu().numpy(), y64[:, 700], rtol=1e-4)
