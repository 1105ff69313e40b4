"""GPU checks of the drop-in modules and host plumbing: PackedLinear's bf16
scales, the reference constructor of the resident expert module, FastRot's
cache, the device rotation tables against the golden fixture, and split-K
workspaces that outlive the graphs captured on them.  Every launch goes
through libvq2_amd.so; the references are the CPU oracle (oracle/)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from compressai_amd import kernels as K, synth
from oracle import vq2_oracle as O
from act_rounding import fp16_row_scaled

pytestmark = pytest.mark.gpu

TOL = 1e-3
GOLDEN = Path(__file__).resolve().parent / "golden" / "rot_tables.npz"


def _rot_np(rot):
    return rot.perm.cpu().numpy(), rot.sign.float().cpu().numpy().astype(np.int8)


def test_packed_linear_rounds_scales_to_bf16(dev):
    """PackedLinear holds bf16 row scales (vq2/runtime.py:78): its output is
    the oracle's with bf16-rounded scales, and measurably not the oracle's
    with the container's fp16 scales."""
    from compressai_amd.runtime import PackedLinear

    n, out = 2048, 2048
    cbs = {"16": synth.codebook(9320).to(dev)}
    m = synth.vq_matrix(9320, out, n, bpw=2)
    lin = PackedLinear((out, n), (16,), "layers.0.self_attn.o_proj", [m["idx0"]], m["scale"], cbs, dev)
    assert lin.scale.dtype == torch.bfloat16
    x = synth.activations(9321, (1, n), dtype=torch.float32)
    y = lin(x.to(dev), out_dtype=torch.float32).cpu().numpy()
    perm, sign = _rot_np(lin.rot)
    xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    _, y_bf = O.vq_gemv(xr, m["idx0"], None, cbs["16"].cpu(), None, m["scale"].to(torch.bfloat16))
    _, y_h = O.vq_gemv(xr, m["idx0"], None, cbs["16"].cpu(), None, m["scale"])
    assert O.max_rel_err(y, y_bf) < 2e-5
    assert O.max_rel_err(y, y_h) > 1e-4


def test_resident_experts_reference_constructor(dev):
    """PackedMoEExpertUniversal(q_gate_up, q_down, cb16, device) built from
    quantized dicts shaped as the reference reads them (256 experts,
    idx[0] viewed as [256, 1024, 256] / [256, 2048, 64], bf16 scales,
    vq2/load_and_test_full_35b.py:31-47), T = 1 and 3, against the oracle."""
    from compressai_amd.moe import PackedMoEExpertUniversal

    E = 256
    gu = synth.indices16(9330, (E * 1024, 256))
    dn = synth.indices16(9331, (E * 2048, 64))
    q_gu = {"idx": [gu], "scale": synth.scales(9332, E * 1024), "cfg": (16,), "tag": "moe_gate_up"}
    q_dn = {"idx": [dn], "scale": synth.scales(9333, E * 2048), "cfg": (16,), "tag": "moe_down"}
    cb = synth.codebook(9334)
    mod = PackedMoEExpertUniversal(q_gu, q_dn, cb.to(dev), dev)
    ph, sh = _rot_np(mod.rot_h)
    pi, si = _rot_np(mod.rot_i)
    gu3, dn3 = gu.view(E, 1024, 256), dn.view(E, 2048, 64)
    gus = q_gu["scale"].view(E, 1024).to(torch.bfloat16)
    dns = q_dn["scale"].view(E, 2048).to(torch.bfloat16)
    for T in (1, 3):
        h = synth.activations(9335 + T, (T, 2048), dtype=torch.bfloat16)
        ids = torch.stack([torch.randperm(E, generator=synth.gen(9340 + t))[:8] for t in range(T)])
        w = torch.softmax(synth.activations(9345 + T, (T, 8)).float(), -1)
        out = mod(h.to(dev), ids.to(dev), w.to(dev))
        assert out.shape == (T, 2048) and out.dtype == torch.bfloat16
        ref = O.moe_experts(h, ids.numpy(), w.numpy(), lambda e: (gu3[e], None, gus[e], dn3[e], None, dns[e]),
                            cb, None, ph, sh.astype(np.float32), pi, si.astype(np.float32))
        # one rounding of the fp32 result to bf16: within one bf16 ulp of each element
        err = np.abs(out.float().cpu().numpy() - ref)
        assert np.all(err <= 2.0 ** -8 * np.abs(ref) + 1e-5 * np.abs(ref).max()), T


def test_fastrot_cache_and_deferred_scale(dev):
    """FastRot (vq2/runtime.py:37-66): the unnormalised RHT (scale 1), the
    same tensor returned while the input is unchanged, recomputed after an
    in-place write; VQ GEMV with rs = RS on its output equals the normalised
    RHT followed by the GEMV."""
    from compressai_amd.rot import RS, FastRot, get_rot

    n = 4096
    rot = get_rot("layers.3.self_attn.q_proj", n, dev)
    fr = FastRot.get("layers.3.self_attn.q_proj", n, dev, rot, out_dtype=torch.float32)
    assert FastRot.get("layers.3.self_attn.q_proj", n, dev, rot) is fr
    perm, sign = _rot_np(rot)
    x = synth.activations(9350, n, dtype=torch.float32).to(dev)
    y1 = fr(x)
    ref1 = O.rht(x.cpu(), perm, sign, 2048, scale=1.0)
    assert O.max_rel_err(y1.cpu().numpy(), ref1) < 1e-5
    assert fr(x) is y1                      # cache hit: same input, same version
    x.mul_(-0.5)                            # in-place write bumps the version
    y2 = fr(x)
    assert y2 is not y1
    assert O.max_rel_err(y2.cpu().numpy(), O.rht(x.cpu(), perm, sign, 2048, scale=1.0)) < 1e-5
    m = synth.vq_matrix(9351, 1024, n, bpw=2)
    cb = synth.codebook(9352)
    y = K.vq_gemv_16(y2, m["idx0"].to(dev), cb.to(dev), m["scale"].to(dev), 1024, n, RS, out_dtype=torch.float32)
    xr = O.rht(x.cpu(), perm, sign, 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], None, cb, None, m["scale"])
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL


def test_rot_tables_on_device_match_golden(dev):
    """The rotations built on this machine (get_rot on the GPU) hold the
    permutation and signs of the committed fixture."""
    from compressai_amd.rot import get_rot

    G = np.load(GOLDEN)
    for tag, n in (("moe_expert_2048", 2048), ("moe_expert_512", 512), ("layers.0.mlp.down_proj", 6144)):
        rot = get_rot(tag, n, dev)
        assert np.array_equal(rot.perm.cpu().numpy(), G[f"{tag}|{n}|perm"].astype(np.int64)), tag
        assert np.array_equal(rot._sign8.cpu().numpy(), G[f"{tag}|{n}|sign"]), tag


def test_small_m_workspace_outlives_captured_graph(dev):
    """A graph captured on the split-K workspace keeps working after a larger
    launch replaces that workspace: the replaced buffer stays alive, so the
    first graph's replays still equal its eager result."""
    cb = synth.codebook(9360).to(dev)
    ma = synth.vq_matrix(9361, 512, 2048, bpw=2)
    mb = synth.vq_matrix(9362, 6144, 2048, bpw=2)
    xa = synth.activations(9363, (8, 2048), dtype=torch.float16).to(dev)
    xb = synth.activations(9364, (64, 2048), dtype=torch.float16).to(dev)
    ia, sa = ma["idx0"].to(dev), ma["scale"].to(dev)
    ib, sb = mb["idx0"].to(dev), mb["scale"].to(dev)
    ya = torch.empty((8, 512), dtype=torch.float32, device=dev)
    yb = torch.empty((64, 6144), dtype=torch.float32, device=dev)
    fa = lambda: K.vq_gemm_small_m(xa, ia, None, cb, None, sa, 512, 2048, y=ya)
    fb = lambda: K.vq_gemm_small_m(xb, ib, None, cb, None, sb, 6144, 2048, y=yb)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        fa()
        ref_a = ya.clone()
        ga = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ga, stream=s):
            fa()
        fb()                                  # needs a larger workspace on the same stream
        ref_b = yb.clone()
        gb = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gb, stream=s):
            fb()
    torch.cuda.synchronize(dev)
    for r in range(3):
        ya.zero_()
        yb.zero_()
        ga.replay()
        gb.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(ya, ref_a), r
        assert torch.equal(yb, ref_b), r
        junk = torch.randn(1 << 20, device=dev)   # eager allocations between the replays
        del junk
    _, y64 = O.vq_gemv(xa.cpu(), ma["idx0"], None, cb.cpu(), None, ma["scale"])
    assert max(O.max_rel_err(ref_a[b].cpu().numpy(), y64[b]) for b in range(8)) < TOL


@pytest.mark.parametrize("cfg,out,n", [((16, 16), 6144, 2048), ((16,), 151936, 2048), ((16, 16), 2048, 6144)])
def test_packed_linear_sorted_layout_batch1(dev, cfg, out, n):
    """Large PackedLinear matrices keep a code-sorted copy of their planes and
    run batch 1 on it (RHT fused in the kernel); batch 2 runs the sorted batch
    kernel (LM head, 6144-wide input) or the gather kernel; the outputs and
    the LM-head top-1 match the oracle."""
    from compressai_amd.runtime import PackedLinear, PackedLMHead

    bpw = 4 if cfg == (16, 16) else 2
    cbs = {"16": synth.codebook(9380).to(dev), "16_16": synth.codebook(9381).to(dev)}
    m = synth.vq_matrix(9382 + out, out, n, bpw=bpw)
    lin = PackedLinear((out, n), cfg, f"t_sorted_{out}_{n}", [m["idx0"], m["idx1"]][:len(cfg)], m["scale"], cbs, dev)
    assert lin.sorted is not None and lin.sorted.has_stage2 == (bpw == 4)
    x = synth.activations(9383, (1, n), dtype=torch.float32)
    y = lin(x.to(dev), out_dtype=torch.float32)
    perm, sign = _rot_np(lin.rot)
    xr = O.rht(x, perm, sign, lin.rot.hb).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cbs["16"].cpu(), cbs["16_16"].cpu() if bpw == 4 else None,
                       lin.scale.cpu())
    assert O.max_rel_err(y.cpu().numpy(), y64) < TOL
    # batch 2: the sorted batch kernel for the LM head and the 6144-wide
    # input (x rotated first, held in fp16 under a power-of-two scale per
    # row), the gather kernel with the RHT built in for the gate shape
    y2 = lin(torch.cat([x, x]).to(dev), out_dtype=torch.float32)
    batch_kernel = out == 151936 or n > 2048
    xk = fp16_row_scaled(lin.rot.fwd(x.to(dev), out_dtype=torch.float32).cpu().numpy()) if batch_kernel else xr
    _, y64k = O.vq_gemv(xk, m["idx0"], m["idx1"], cbs["16"].cpu(), cbs["16_16"].cpu() if bpw == 4 else None,
                        lin.scale.cpu())
    for b in range(2):
        assert O.max_rel_err(y2[b].cpu().numpy(), y64[0]) < TOL
        assert O.max_rel_err(y2[b].cpu().numpy(), y64k[0]) < 1e-5
    if cfg == (16,):
        idx, val = PackedLMHead(lin).argmax(x.to(dev))
        assert int(idx[0]) == int(np.argmax(y64[0]))
        assert abs(float(val[0]) - y64[0].max()) <= 1e-5 * abs(y64[0].max())


@pytest.mark.parametrize("cfg", [(16,), (16, 16)])
def test_packed_linear_release_planes(dev, cfg):
    """release_planes() frees the reference planes and keeps only the
    code-sorted copy: batch 1 on the sorted GEMV, batch 2, 3 and 6 on the
    sorted batch kernel in groups of up to 4 rows, and the top-1 of
    PackedLMHead; outputs match the oracle on the activation as each kernel
    holds it (to 1e-5), and the resident bytes drop by the planes."""
    from compressai_amd.runtime import PackedLinear, PackedLMHead

    out, n = 4096, 2048
    bpw = 4 if cfg == (16, 16) else 2
    cbs = {"16": synth.codebook(9400).to(dev), "16_16": synth.codebook(9401).to(dev)}
    m = synth.vq_matrix(9402 + bpw, out, n, bpw=bpw)
    lin = PackedLinear((out, n), cfg, f"t_release_{bpw}", [m["idx0"], m["idx1"]][:len(cfg)], m["scale"], cbs, dev)
    assert lin.sorted is not None and not lin.planes_released
    before = lin.nbytes()
    lin.release_planes()
    assert lin.planes_released and lin.idx0 is None
    assert before - lin.nbytes() == out * (n // 8) * 2 * len(cfg)
    cb1 = cbs["16_16"].cpu() if bpw == 4 else None
    for B in (1, 2, 3, 6):
        x = synth.activations(9405 + B, (B, n), dtype=torch.float32)
        y = lin(x.to(dev), out_dtype=torch.float32)
        assert y.shape == (B, out)
        xr = lin.rot.fwd(x.to(dev), out_dtype=torch.float32).cpu().numpy()
        xk = xr if B == 1 else fp16_row_scaled(xr)
        _, y64 = O.vq_gemv(xk, m["idx0"], m["idx1"], cbs["16"].cpu(), cb1, lin.scale.cpu())
        for b in range(B):
            assert O.max_rel_err(y[b].cpu().numpy(), y64[b]) < 1e-5, (B, b)
        if cfg == (16,):
            idx, val = PackedLMHead(lin).argmax(x.to(dev))
            assert idx.cpu().tolist() == [int(np.argmax(y64[b])) for b in range(B)], B


def test_packed_linear_16_8_on_the_sorted_layout(dev):
    """A (16,8) 3 bpw PackedLinear of 2.1 M codes keeps a sorted copy whose
    stage 2 is the uint8 plane (packed as codes below 256 into the [256, 8]
    stage-2 codebook) and runs batch 1 on it with the RHT fused; the output
    matches the oracle and the gather kernel on the reference planes."""
    from compressai_amd import kernels as K
    from compressai_amd.runtime import PackedLinear

    out, n = 4096, 2048
    cbs = {"16": synth.codebook(9390).to(dev), "16_8": synth.codebook(9391, 256).to(dev)}
    m = synth.vq_matrix(9392, out, n, bpw=3)
    lin = PackedLinear((out, n), (16, 8), "t_sorted_16_8", [m["idx0"], m["idx1"]], m["scale"], cbs, dev)
    assert lin.sorted is not None and lin.sorted.s2_kind == 2
    x = synth.activations(9393, (1, n), dtype=torch.float32)
    y = lin(x.to(dev), out_dtype=torch.float32)
    perm, sign = _rot_np(lin.rot)
    xr = O.rht(x, perm, sign, lin.rot.hb).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cbs["16"].cpu(), cbs["16_8"].cpu(), lin.scale.cpu())
    assert O.max_rel_err(y.cpu().numpy(), y64) < TOL
    yg = K.vq_gemv(torch.from_numpy(xr).to(dev), lin.idx0, lin.idx1, cbs["16"], cbs["16_8"], lin.scale, out, n,
                   out_dtype=torch.float32)
    assert O.max_rel_err(y.cpu().numpy(), yg.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("B", [2, 3, 4])
def test_lm_head_batch_top1_on_sorted_batch_kernel(dev, B):
    """An LM head of 32768 x 2048 (8.4 M codes) at batch 2-4: PackedLMHead.argmax
    and the logits of PackedLinear run the sorted batch kernel after the RHT;
    the top-1 of every row is the argmax of the oracle's logits of the
    activation as the kernel holds it, and the logits match them."""
    from compressai_amd.runtime import PackedLinear, PackedLMHead

    out, n = 32768, 2048
    cbs = {"16": synth.codebook(9386).to(dev)}
    m = synth.vq_matrix(9387, out, n, bpw=2)
    lin = PackedLinear((out, n), (16,), "lm_head", [m["idx0"]], m["scale"], cbs, dev)
    assert lin._sorted_batch_ok(B, cbs["16"])
    x = synth.activations(9388 + B, (B, n), dtype=torch.float16)
    # the activation as the kernel holds it: the rotation the runtime ran
    # (pinned against the oracle by the RHT tests), rounded as the kernel rounds
    xk = fp16_row_scaled(lin.rot.fwd(x.to(dev), out_dtype=torch.float32).cpu().numpy())
    _, y64k = O.vq_gemv(xk, m["idx0"], None, cbs["16"].cpu(), None, lin.scale.cpu())
    idx, val = PackedLMHead(lin).argmax(x.to(dev))
    y = lin(x.to(dev), out_dtype=torch.float32)
    for b in range(B):
        assert int(idx[b]) == int(np.argmax(y64k[b])), b
        assert abs(float(val[b]) - y64k[b].max()) <= 1e-5 * abs(y64k[b].max()), b
        assert O.max_rel_err(y[b].cpu().numpy(), y64k[b]) < 1e-5, b


@pytest.mark.parametrize("act", [torch.float32, torch.float16])
def test_packed_projections_qkv(dev, act):
    """q, k and v of a 2048-wide attention (tag "attn", one activation) in one
    launch: the sorted layout at batch 1 (0.79 M codes together), the fused
    gather kernel at batch 2, the sorted batch kernel at batch 3 (activation
    held in fp16 under a power-of-two scale per row); every output matches
    the oracle (to 1e-5 on the activation as the kernel holds it) and the
    projection's own PackedLinear forward."""
    from compressai_amd.runtime import PackedLinear, PackedProjections

    n = 2048
    cbs = {"16": synth.codebook(9390).to(dev)}
    lins = []
    mats = []
    for k, out in enumerate((2048, 512, 512)):
        m = synth.vq_matrix(9391 + k, out, n, bpw=2)
        mats.append(m)
        lins.append(PackedLinear((out, n), (16,), "attn", [m["idx0"]], m["scale"], cbs, dev))
    # q (2^19 codes) holds sorted planes of its own, k and v (2^17) do not
    assert lins[0].sorted is not None and all(lin.sorted is None for lin in lins[1:])
    proj = PackedProjections(lins)
    assert proj.sorted is not None and len(proj.sorted) == 3
    # one launch of 0.79 M codes: chunks of the launch's height for all three
    R = K.sorted_launch_rows_per_chunk([2048, 512, 512], n // 8, dev)
    assert R is not None and all(sp.rows_per_chunk == R for sp in proj.sorted)
    perm, sign = _rot_np(lins[0].rot)
    for B in (1, 2, 3):
        x = synth.activations(9395 + B, (B, n), dtype=act)
        ys = proj(x.to(dev), out_dtype=torch.float32)
        xr = O.rht(x.float(), perm, sign, 2048).astype(np.float32)
        xk = fp16_row_scaled(lins[0].rot.fwd(x.to(dev), out_dtype=torch.float32).cpu().numpy()) if B >= 3 else xr
        for lin, m, y in zip(lins, mats, ys):
            assert y.shape == (B, lin.out) and y.dtype == torch.float32
            own = lin(x.to(dev), out_dtype=torch.float32)
            assert O.max_rel_err(y.cpu().numpy(), own.cpu().numpy()) < (1e-5 if B <= 2 else TOL)
            _, y64 = O.vq_gemv(xr, m["idx0"], None, cbs["16"].cpu(), None, lin.scale.cpu())
            assert O.max_rel_err(y.cpu().numpy(), y64) < TOL
            _, y64k = O.vq_gemv(xk, m["idx0"], None, cbs["16"].cpu(), None, lin.scale.cpu())
            assert O.max_rel_err(y.cpu().numpy(), y64k) < 1e-5


@pytest.mark.parametrize("B", [2, 4])
def test_packed_projections_gate_up_batch(dev, B):
    """gate and up (tag "mlp", 2 x 6144 x 2048 at 4 bpw, 6.3 M codes) as one
    PackedProjections at batch 2 and 4: one sorted batch launch after the
    RHT; each output matches the oracle, to 1e-5 on the activation as the
    kernel holds it."""
    from compressai_amd.runtime import PackedLinear, PackedProjections

    n = 2048
    cbs = {"16": synth.codebook(9400).to(dev), "16_16": synth.codebook(9401).to(dev)}
    ms = [synth.vq_matrix(9402 + k, 6144, n, bpw=4) for k in range(2)]
    lins = [PackedLinear((6144, n), (16, 16), "mlp", [m["idx0"], m["idx1"]], m["scale"], cbs, dev) for m in ms]
    proj = PackedProjections(lins)
    assert proj.sorted is not None and proj.codes >= 2 << 20
    x = synth.activations(9405 + B, (B, n), dtype=torch.float16)
    ys = proj(x.to(dev), out_dtype=torch.float32)
    perm, sign = _rot_np(lins[0].rot)
    xr = O.rht(x.float(), perm, sign, 2048).astype(np.float32)
    xk = fp16_row_scaled(lins[0].rot.fwd(x.to(dev), out_dtype=torch.float32).cpu().numpy())
    for lin, m, y in zip(lins, ms, ys):
        assert y.shape == (B, 6144)
        args = (m["idx0"], m["idx1"], cbs["16"].cpu(), cbs["16_16"].cpu(), lin.scale.cpu())
        _, y64 = O.vq_gemv(xr, *args)
        _, y64k = O.vq_gemv(xk, *args)
        assert O.max_rel_err(y.cpu().numpy(), y64) < TOL
        assert O.max_rel_err(y.cpu().numpy(), y64k) < 1e-5


def test_packed_projections_rejects_mixed(dev):
    """Projections of other widths, tags or codebooks cannot share a launch."""
    from compressai_amd.runtime import PackedLinear, PackedProjections

    cbs = {"16": synth.codebook(9397).to(dev)}
    other = {"16": synth.codebook(9398).to(dev)}
    m = synth.vq_matrix(9399, 512, 2048, bpw=2)
    a = PackedLinear((512, 2048), (16,), "attn", [m["idx0"]], m["scale"], cbs, dev)
    b = PackedLinear((512, 2048), (16,), "mlp", [m["idx0"]], m["scale"], cbs, dev)
    c = PackedLinear((512, 2048), (16,), "attn", [m["idx0"]], m["scale"], other, dev)
    for bad in ([a, b], [a, c], [a] * 5):
        with pytest.raises(K.Vq2Error):
            PackedProjections(bad)


def test_function_entries_use_a_sorted_copy_of_large_planes(dev):
    """vq_gemv_16 / vq_gemv_16_16 (the function-level drop-in) at batch 1 on a
    plane of >= 2 M codes keep a code-sorted copy of it: the first call packs
    it, later calls on the same tensor reuse it, an in-place write to the
    plane makes a fresh copy, a freed plane drops its copy, and the results
    match the oracle and the gather kernel."""
    import gc

    out, n = 8192, 2048
    cb = synth.codebook(9395).to(dev)
    cb1 = synth.codebook(9396).to(dev)
    m = synth.vq_matrix(9397, out, n, bpw=4)
    i0, i1, sc = m["idx0"].to(dev), m["idx1"].to(dev), m["scale"].to(dev)
    xr = synth.activations(9398, n, dtype=torch.bfloat16).to(dev)
    K.sorted_cache_enabled(True)
    before = len(K._SORTED_CACHE)
    y = K.vq_gemv_16_16(xr, i0, i1, cb, cb1, sc, out, n, out_dtype=torch.float32)
    assert len(K._SORTED_CACHE) == before + 1
    sp = K._SORTED_CACHE[id(i0)][4]
    y2 = K.vq_gemv_16_16(xr, i0, i1, cb, cb1, sc, out, n, out_dtype=torch.float32)
    assert K._SORTED_CACHE[id(i0)][4] is sp and torch.equal(y, y2)
    _, y64 = O.vq_gemv(xr.float().cpu()[None], m["idx0"], m["idx1"], cb.cpu(), cb1.cpu(), m["scale"])
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL
    yg = K.vq_gemv(xr, i0, i1, cb, cb1, sc, out, n, out_dtype=torch.float32)   # the gather kernel
    assert O.max_rel_err(y.cpu().numpy(), yg.cpu().numpy()) < 1e-5
    # an in-place write: a new copy, and the new codes are used
    i0[0, :8] = 0
    y3 = K.vq_gemv_16_16(xr, i0, i1, cb, cb1, sc, out, n, out_dtype=torch.float32)
    assert K._SORTED_CACHE[id(i0)][4] is not sp
    yg3 = K.vq_gemv(xr, i0, i1, cb, cb1, sc, out, n, out_dtype=torch.float32)
    assert O.max_rel_err(y3.cpu().numpy(), yg3.cpu().numpy()) < 1e-5
    # a 2 bpw plane through vq_gemv_16, bf16 out as the reference returns it
    m2 = synth.vq_matrix(9399, 16384, n, bpw=2)
    j0, s2 = m2["idx0"].to(dev), m2["scale"].to(dev)
    yb = K.vq_gemv_16(xr, j0, cb, s2, 16384, n)
    assert yb.dtype == torch.bfloat16 and id(j0) in K._SORTED_CACHE
    _, yb64 = O.vq_gemv(xr.float().cpu()[None], m2["idx0"], None, cb.cpu(), None, m2["scale"])
    assert O.max_rel_err(yb.float().cpu().numpy(), yb64[0]) < 2.0 ** -8 + TOL
    # freed planes drop their copies; small planes never get one
    k0 = id(i0)
    del i0, j0
    gc.collect()
    assert k0 not in K._SORTED_CACHE
    small = synth.vq_matrix(9400, 256, n, bpw=2)
    K.vq_gemv_16(xr, small["idx0"].to(dev), cb, small["scale"].to(dev), 256, n)
    assert K.sorted_cache_bytes() >= 0 and len(K._SORTED_CACHE) == before
