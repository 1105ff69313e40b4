"""GPU parity of the MoE experts over code-sorted expert pools
(vq2_sorted_moe through the C ABI: gate_up with the RHT built in, down with
SwiGLU + RHT in its prologue, combine) against the fp64 oracle on the same
seeded inputs: ids given (int32 / int64) and the router built in, T = 1..8
(gate_up and down in one launch) and T = 15 (135 pairs: two launches), fp16 / bf16 codebooks and activations, 1 to 9 slices per chunk, NaN for an
expert id outside the pool, bit-identical repeats, and agreement with the
gather kernels on the reference pools.

Tolerance: max_i |y_i - ref_i| / max_i |ref_i| <= 1e-3 (the decode-path
contract); observed ~1e-6 (fp32 accumulation in another order)."""
import numpy as np
import pytest
import torch

from compressai_amd import kernels as K, synth
from oracle import vq2_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _pools(seed, E):
    gu = synth.indices16(seed + 2, (E, 1024, 256))
    gus = synth.scales(seed + 3, (E, 1024))
    dn = synth.indices16(seed + 12, (E, 2048, 64))
    dns = synth.scales(seed + 13, (E, 2048))
    return gu, gus, dn, dns


def _rot_np(rot):
    return rot.perm.cpu().numpy(), rot.sign.float().cpu().numpy()


def _module(dev, seed, E, cb_dtype=torch.float16, sorted_layout=True):
    from compressai_amd.moe import ResidentMoEExperts

    cb = synth.codebook(seed, dtype=cb_dtype)
    gu, gus, dn, dns = _pools(seed, E)
    mod = ResidentMoEExperts.from_pools(gu.to(dev), gus.to(dev), dn.to(dev), dns.to(dev), cb.to(dev),
                                        out_dtype=torch.float32, sorted_layout=sorted_layout)
    return mod, cb, gu, gus, dn, dns


def _oracle(mod, h, ids, w, cb, gu, gus, dn, dns):
    ph, sh = _rot_np(mod.rot_h)
    pi, si = _rot_np(mod.rot_i)
    return O.moe_experts(h, ids, w, lambda e: (gu[e], None, gus[e], dn[e], None, dns[e]), cb, None, ph, sh, pi, si)


@pytest.mark.parametrize("T,P,ids_dtype,h_dtype", [
    (1, 9, torch.int32, torch.float16),
    (2, 8, torch.int64, torch.bfloat16),
    (3, 3, torch.int32, torch.float32),
    (8, 9, torch.int64, torch.float16),
    (15, 9, torch.int32, torch.float32),
])
def test_sorted_moe_experts_vs_oracle(dev, T, P, ids_dtype, h_dtype):
    E = 24
    mod, cb, gu, gus, dn, dns = _module(dev, 9600 + T, E)
    assert mod.sorted_gu is not None and mod.sorted_gu.rows_per_chunk == 205 and mod.sorted_dn.chunks == 9
    h = synth.activations(9601 + T, (T, 2048), dtype=h_dtype)
    ids = torch.stack([torch.randperm(E, generator=synth.gen(9610 + t))[:P] for t in range(T)]).to(ids_dtype)
    w = torch.softmax(synth.activations(9620 + T, (T, P)).float(), -1)
    out = mod.experts(h.to(dev), ids.to(dev), w.to(dev))
    assert out.shape == (T, 2048) and out.dtype == torch.float32
    ref = _oracle(mod, h, ids.numpy(), w.numpy(), cb, gu, gus, dn, dns)
    assert O.max_rel_err(out.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("T,slices", [(3, None), (3, (2, 1)), (3, (3, 2)), (15, None)])
def test_sorted_moe_tall_down_pool(dev, T, slices):
    """The down pool in taller chunks (5 of 410 rows, 16-bit positions, rows
    summed in 512-thread halves), which the module runs from T = 2 on: the
    oracle's result, bit-identical on repeated calls, in one launch (T = 3)
    and in three (T = 15: 135 pairs); T = 1 keeps the default chunks, and
    release_tall_down() returns every T to them."""
    E, P = 12, 9
    mod, cb, gu, gus, dn, dns = _module(dev, 9750, E)
    tall = mod.sorted_dn_tall
    assert tall is not None and tall.rows_per_chunk == 410 and tall.chunks == 5
    assert mod._down_pool(1) is mod.sorted_dn and mod._down_pool(2) is tall
    h = synth.activations(9751 + T, (T, 2048), dtype=torch.float16).to(dev)
    ids = torch.stack([torch.randperm(E, generator=synth.gen(9760 + t))[:P] for t in range(T)]).to(torch.int32).to(dev)
    w = torch.softmax(synth.activations(9770 + T, (T, P)).float(), -1).to(dev)
    rh, ri = mod._rots()
    run = lambda: K.vq_sorted_moe(h, mod.sorted_gu, mod.gate_up_scale, tall, mod.down_scale, mod.cb16, rh, ri,
                                  ids=ids, w=w, slices=slices)
    a = run()
    b = run()
    assert torch.equal(a, b)
    ref = _oracle(mod, h.cpu(), ids.cpu().numpy(), w.cpu().numpy(), cb, gu, gus, dn, dns)
    assert O.max_rel_err(a.cpu().numpy(), ref) < TOL
    if slices is None:
        assert torch.equal(mod.experts(h, ids, w), a)
    mod.release_tall_down()
    assert mod.sorted_dn_tall is None and mod._down_pool(8) is mod.sorted_dn


@pytest.mark.parametrize("slices", [(1, 1), (3, 2), (7, 4), (2, 5), (9, 9)])
def test_sorted_moe_slices_and_determinism(dev, slices):
    """Every slice count gives the oracle's result (the combine adds up to
    81 shares per row here); repeated calls are bit-identical (fixed
    summation orders)."""
    E, T, P = 12, 2, 9
    mod, cb, gu, gus, dn, dns = _module(dev, 9700, E)
    h = synth.activations(9701, (T, 2048), dtype=torch.float16).to(dev)
    ids = torch.tensor([[3, 0, 11, 7, 1, 2, 4, 6, 8], [5, 3, 2, 9, 10, 0, 1, 11, 7]], dtype=torch.int32).to(dev)
    w = torch.softmax(synth.activations(9702, (T, P)).float(), -1).to(dev)
    rh, ri = mod._rots()
    run = lambda: K.vq_sorted_moe(h, mod.sorted_gu, mod.gate_up_scale, mod.sorted_dn, mod.down_scale, mod.cb16, rh,
                                  ri, ids=ids, w=w, slices=slices)
    a = run()
    b = run()
    assert torch.equal(a, b)
    ref = _oracle(mod, h.cpu(), ids.cpu().numpy(), w.cpu().numpy(), cb, gu, gus, dn, dns)
    assert O.max_rel_err(a.cpu().numpy(), ref) < TOL


def test_sorted_moe_matches_gather_kernels(dev):
    """The sorted pools and the reference pools (gather kernels) agree to
    fp32 accumulation-order rounding, bf16 codebook."""
    E, T, P = 20, 3, 9
    mod, cb, gu, gus, dn, dns = _module(dev, 9750, E, cb_dtype=torch.bfloat16)
    ref_mod = _module(dev, 9750, E, cb_dtype=torch.bfloat16, sorted_layout=False)[0]
    h = synth.activations(9751, (T, 2048), dtype=torch.bfloat16).to(dev)
    ids = torch.stack([torch.randperm(E, generator=synth.gen(9752 + t))[:P] for t in range(T)]).to(dev)
    w = torch.softmax(synth.activations(9760, (T, P)).float(), -1).to(dev)
    a = mod.experts(h, ids, w)
    b = ref_mod.experts(h, ids, w)
    assert O.max_rel_err(a.cpu().numpy(), b.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("T,slices", [(1, (5, 3)), (8, (2, 1)), (4, (3, 6))])
def test_sorted_moe_fresh_inputs_back_to_back(dev, T, slices):
    """Ten layers back to back on one stream, each with other activations,
    experts and weights and no synchronisation in between (the workspace of
    partials and shares is reused by every layer): a value left from the
    previous layer would show far above the tolerance.  Each output matches
    the gather kernels on the reference pools."""
    E, P = 40, 9
    mod, cb, gu, gus, dn, dns = _module(dev, 9770, E)
    ref_mod = _module(dev, 9770, E, sorted_layout=False)[0]
    rh, ri = mod._rots()
    cases = []
    for i in range(10):
        h = synth.activations(9771 + i, (T, 2048), dtype=torch.float16).to(dev)
        ids = torch.stack([torch.randperm(E, generator=synth.gen(9790 + 10 * i + t))[:P] for t in range(T)]).to(dev)
        w = torch.softmax(synth.activations(9880 + i, (T, P)).float(), -1).to(dev)
        cases.append((h, ids, w))
    outs = [K.vq_sorted_moe(h, mod.sorted_gu, mod.gate_up_scale, mod.sorted_dn, mod.down_scale, mod.cb16, rh, ri,
                            ids=ids, w=w, slices=slices) for h, ids, w in cases]
    torch.cuda.synchronize(dev)
    for i, ((h, ids, w), out) in enumerate(zip(cases, outs)):
        ref = ref_mod.experts(h, ids, w)
        assert O.max_rel_err(out.cpu().numpy(), ref.cpu().numpy()) < 1e-5, i


@pytest.mark.parametrize("H,I", [(1024, 256), (4096, 1024)])
def test_sorted_moe_other_widths_vs_oracle(dev, H, I):
    """Widths other than the 2048 / 512 of the reference model take the
    general prologues (one 2048-point block for h and one 512-point block for
    the intermediate have prologues of their own): hidden 1024 (one 1024-point
    block) and 4096 (two 2048-point blocks), intermediate 256 and 1024."""
    from compressai_amd.moe import ResidentMoEExperts

    E, T, P = 6, 2, 3
    cb = synth.codebook(9950)
    gu = synth.indices16(9951, (E, 2 * I, H // 8))
    gus = synth.scales(9952, (E, 2 * I))
    dn = synth.indices16(9953, (E, H, I // 8))
    dns = synth.scales(9954, (E, H))
    mod = ResidentMoEExperts.from_pools(gu.to(dev), gus.to(dev), dn.to(dev), dns.to(dev), cb.to(dev),
                                        out_dtype=torch.float32)
    assert mod.sorted_gu is not None
    assert mod.rot_h.hb == min(2048, H) and mod.rot_i.hb == min(2048, I)
    h = synth.activations(9955, (T, H), dtype=torch.float16)
    ids = torch.tensor([[0, 5, 2], [4, 1, 3]], dtype=torch.int32)
    w = torch.softmax(synth.activations(9956, (T, P)).float(), -1)
    out = mod.experts(h.to(dev), ids.to(dev), w.to(dev))
    ref = _oracle(mod, h, ids.numpy(), w.numpy(), cb, gu, gus, dn, dns)
    assert O.max_rel_err(out.cpu().numpy(), ref) < TOL


def test_sorted_moe_bad_expert_id_gives_nan_token(dev):
    """An id outside the pool (E, or negative) makes its token's output NaN
    and leaves the other tokens exact."""
    E, T, P = 6, 3, 2
    mod, cb, gu, gus, dn, dns = _module(dev, 9800, E)
    h = synth.activations(9801, (T, 2048), dtype=torch.float16)
    ids = torch.tensor([[1, 4], [E, 2], [3, -1]], dtype=torch.int64)
    w = torch.tensor([[0.5, 0.5], [0.25, 0.75], [1.0, 2.0]], dtype=torch.float32)
    out = mod.experts(h.to(dev), ids.to(dev), w.to(dev)).cpu()
    assert torch.isnan(out[1]).all() and torch.isnan(out[2]).all()
    ref = _oracle(mod, h[:1], ids[:1].numpy(), w[:1].numpy(), cb, gu, gus, dn, dns)
    assert O.max_rel_err(out[:1].numpy(), ref) < TOL


@pytest.mark.parametrize("T", [1, 5])
def test_sorted_moe_router_ids_and_weights(dev, T):
    """Router built into the sorted gate_up launch: the published ids and
    weights equal the standalone router's bit for bit and the oracle's
    router (softmax, top-k, renormalised, ties to the lower id; the shared
    expert's sigmoid gate), and the layer output equals the same experts run
    with those ids."""
    from compressai_amd.moe import MoELayer

    E, k = 64, 6
    cb = synth.codebook(9900)
    gu, gus, dn, dns = _pools(9900, E + 1)
    gate = synth.activations(9901, 2048) * 0.02
    layer = MoELayer(gu.to(dev), gus.to(dev), dn.to(dev), dns.to(dev), cb.to(dev), gate.to(dev), top_k=k)
    m = layer.experts_mod
    h = synth.activations(9902, (T, 2048), dtype=torch.float16).to(dev)
    logits = synth.activations(9903, (T, E), dtype=torch.float16).to(dev)
    rh, ri = m._rots()
    # the down pool the layer runs for T tokens (the taller chunks from T = 2 on)
    out, ids, w = K.vq_sorted_moe(h, m.sorted_gu, m.gate_up_scale, m._down_pool(T), m.down_scale, m.cb16, rh, ri,
                                  logits=logits, top_k=k, shared_id=E, shared_gate=layer.shared_gate)
    rid, rw = layer.route(h, logits)
    assert torch.equal(ids.cpu(), rid.cpu().to(torch.int32))
    assert torch.equal(w.cpu(), rw.cpu())
    oid, ow = O.router_topk(logits.float().cpu().numpy(), k)
    assert ids.cpu()[:, :k].numpy().tolist() == oid.tolist()
    assert np.allclose(w.cpu()[:, :k].numpy(), ow, rtol=1e-5, atol=1e-7)
    assert (ids.cpu()[:, k] == E).all()
    sg = 1 / (1 + np.exp(-(h.double().cpu().numpy() @ gate.double().numpy())))
    assert np.allclose(w.cpu()[:, k].numpy(), sg, rtol=1e-5)
    again = m.experts(h, rid, rw)
    assert torch.equal(out, again)
    assert torch.equal(layer(h, logits), out)


@pytest.mark.parametrize("T,P", [(1, 4), (3, 5)])
def test_sorted_moe_16_8_pools_vs_oracle(dev, T, P):
    """Promoted 3 bpw (16,8) experts on two-stage sorted pools: stage-1
    entries gather from the 65536-row codebook, stage-2 entries from the
    [256, 8] stage-2 codebook; gate_up and down in one launch, then the
    combine, against the fp64 oracle."""
    from compressai_amd.rot import get_rot

    E = 6
    cb = synth.codebook(9980)
    cb8 = synth.codebook(9981, 256)
    gu, gus, dn, dns = _pools(9980, E)
    g8 = synth.gen(9982)
    gu1 = torch.randint(0, 256, (E, 1024, 256), generator=g8, dtype=torch.int32).to(torch.uint8)
    dn1 = torch.randint(0, 256, (E, 2048, 64), generator=g8, dtype=torch.int32).to(torch.uint8)
    gup = K.SortedPool(gu, device=dev, idx1=gu1)
    dnp = K.SortedPool(dn, device=dev, idx1=dn1)
    assert gup.s2_kind == 2 and dnp.s2_kind == 2
    rh, ri = get_rot("moe_expert_2048", 2048, dev), get_rot("moe_expert_512", 512, dev)
    h = synth.activations(9983 + T, (T, 2048), dtype=torch.float16)
    ids = torch.stack([torch.randperm(E, generator=synth.gen(9984 + t))[:P] for t in range(T)]).to(torch.int32)
    w = torch.softmax(synth.activations(9990 + T, (T, P)).float(), -1)
    out = K.vq_sorted_moe(h.to(dev), gup, gus.to(dev), dnp, dns.to(dev), cb.to(dev),
                          (rh._perm32, rh._sign8, rh.hb, rh.scale), (ri._perm32, ri._sign8, ri.hb, ri.scale),
                          ids=ids.to(dev), w=w.to(dev), cb1=cb8.to(dev))
    ref = O.moe_experts(h, ids.numpy(), w.numpy(), lambda e: (gu[e], gu1[e], gus[e], dn[e], dn1[e], dns[e]), cb, cb8,
                        *_rot_np(rh), *_rot_np(ri))
    assert O.max_rel_err(out.cpu().numpy(), ref) < TOL
    with pytest.raises(K.Vq2Error):  # a two-stage pool without its codebook
        K.vq_sorted_moe(h.to(dev), gup, gus.to(dev), dnp, dns.to(dev), cb.to(dev),
                        (rh._perm32, rh._sign8, rh.hb, rh.scale), (ri._perm32, ri._sign8, ri.hb, ri.scale),
                        ids=ids.to(dev), w=w.to(dev))
