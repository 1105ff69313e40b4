"""GPU parity of the batch 1-4 VQ GEMM over the code-sorted layout
(vq2_sorted_gemm_batch / _argmax through the C ABI) against the fp64 oracle
on the same seeded inputs: 2 and 4 bpw, fp16 / bf16 codebooks, fp32 / fp16 /
bf16 activations, the config 2 / 3 shapes and ragged ones, one or several
workgroups per chunk, two matrices per launch, the fused top-1 at the
config 3 LM-head size (ties resolve to the lower row), graph replays and the
error paths.

Tolerance: max_i |y_i - ref_i| / max_i |ref_i| <= 1e-3 against the fp32
activation (the decode-path contract; the kernel holds the activation in
fp16 under a power-of-two scale per row, ~1e-4 observed), and <= 1e-5
against the oracle fed that same rounded activation (fp32 accumulation in
another order, ~1e-7 observed), which pins the rounding to exactly that."""
import numpy as np
import pytest
import torch

from compressai_amd import kernels as K, synth
from compressai_amd.kernels import Vq2Error
from oracle import vq2_oracle as O
from act_rounding import fp16_row_scaled as _fp16_scaled

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_ROUNDED = 1e-5


def _mk(seed, rows, n, bpw, dev, cb_dtype=torch.float16):
    m = synth.vq_matrix(seed, rows, n, bpw=bpw)
    cb0 = synth.codebook(seed + 1, dtype=cb_dtype)
    cb1 = synth.codebook(seed + 2, dtype=cb_dtype) if bpw == 4 else None
    sp = K.SortedPlanes(m["idx0"], m["idx1"], rows, n, device=dev)
    return m, cb0, cb1, sp


def _x(seed, B, n, dtype):
    x = synth.activations(seed, (B, n), dtype=torch.float32) * 0.5
    return x.to(dtype)


@pytest.mark.parametrize("rows,n,bpw,B,x_dtype,slices", [
    (2048, 2048, 2, 4, torch.float32, None),     # o / configs[0] shape
    (6144, 2048, 4, 3, torch.float16, None),     # gate / up
    (2048, 6144, 4, 2, torch.bfloat16, None),    # down (62-row chunks)
    (1000, 512, 2, 4, torch.float32, 3),
    (97, 800, 2, 2, torch.float32, 1),           # ng = 100: not a power of two
    (517, 2048, 4, 1, torch.float16, 7),
    (300, 2048, 2, 4, torch.float32, 64),        # more slices than iterations per chunk
])
def test_batch_gemm_vs_oracle(dev, rows, n, bpw, B, x_dtype, slices):
    m, cb0, cb1, sp = _mk(9700 + rows + n, rows, n, bpw, dev)
    x = _x(9701 + rows, B, n, x_dtype)
    (y,) = K.vq_sorted_gemm_batch(x.to(dev), [(sp, m["scale"].to(dev))], cb0.to(dev),
                                  None if cb1 is None else cb1.to(dev), n, slices=slices)
    assert y.shape == (B, rows) and y.dtype == torch.float32
    xf = x.float().numpy()
    _, y64 = O.vq_gemv(xf, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    _, y64r = O.vq_gemv(_fp16_scaled(xf), m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    got = y.cpu().numpy()
    for b in range(B):
        assert O.max_rel_err(got[b], y64[b]) < TOL, b
        assert O.max_rel_err(got[b], y64r[b]) < TOL_ROUNDED, b


def test_batch_gemm_bf16_codebook_scale_rs_and_outputs(dev):
    rows, n, B = 1536, 2048, 4
    m, cb0, cb1, sp = _mk(9720, rows, n, 4, dev, cb_dtype=torch.bfloat16)
    sc = m["scale"].to(torch.bfloat16)
    x = _x(9721, B, n, torch.float32)
    (y,) = K.vq_sorted_gemm_batch(x.to(dev), [(sp, sc.to(dev))], cb0.to(dev), cb1.to(dev), n, rs=0.25,
                                  out_dtype=torch.bfloat16)
    _, y64r = O.vq_gemv(_fp16_scaled(x.numpy()), m["idx0"], m["idx1"], cb0, cb1, sc, rs=0.25)
    err = np.abs(y.float().cpu().numpy() - y64r)
    assert np.all(err <= 2.0 ** -8 * np.abs(y64r) + 1e-5 * np.abs(y64r).max())  # one bf16 rounding


def test_batch_gemm_two_matrices_and_determinism(dev):
    """gate and up in one launch, each equal to the oracle, and the launch
    equal to itself bit for bit over repeated calls."""
    n, B = 2048, 4
    ms = [_mk(9730 + k, 6144, n, 4, dev) for k in range(2)]
    cb0, cb1 = ms[0][1], ms[0][2]
    x = _x(9735, B, n, torch.float16)
    mats = [(sp, m["scale"].to(dev)) for m, _, _, sp in ms]
    ys = K.vq_sorted_gemm_batch(x.to(dev), mats, cb0.to(dev), cb1.to(dev), n)
    first = [y.clone() for y in ys]
    for _ in range(3):
        again = K.vq_sorted_gemm_batch(x.to(dev), mats, cb0.to(dev), cb1.to(dev), n)
        assert all(torch.equal(a, b) for a, b in zip(first, again))
    for (m, _, _, _), y in zip(ms, first):
        _, y64 = O.vq_gemv(x.float().numpy(), m["idx0"], m["idx1"], cb0, cb1, m["scale"])
        assert O.max_rel_err(y.cpu().numpy(), y64) < TOL_ROUNDED


def test_batch_gemm_fresh_inputs_back_to_back(dev):
    """Several-slice launches back to back with new activations and no
    synchronisation: the arrival counters return to zero after every call."""
    rows, n = 3000, 2048
    m, cb0, _, sp = _mk(9740, rows, n, 2, dev)
    xs = [_x(9741 + i, 1 + i % 4, n, torch.float32) for i in range(6)]
    outs = [K.vq_sorted_gemm_batch(x.to(dev), [(sp, m["scale"].to(dev))], cb0.to(dev), None, n, slices=5)[0]
            for x in xs]
    for x, y in zip(xs, outs):
        _, y64r = O.vq_gemv(_fp16_scaled(x.numpy()), m["idx0"], None, cb0, None, m["scale"])
        assert O.max_rel_err(y.cpu().numpy(), y64r) < TOL_ROUNDED


@pytest.mark.parametrize("B", [2, 4])
def test_batch_argmax_lm_head_full_size(dev, B):
    """configs[2] LM head 151936 x 2048 at 2 bpw, batch 2 / 4: the fused
    top-1 of every row is the oracle's argmax of the logits of the rounded
    activation, within 1e-3 of the maximum of the fp32-activation logits."""
    rows, n = 151936, 2048
    m, cb0, _, sp = _mk(9750, rows, n, 2, dev)
    x = _x(9751 + B, B, n, torch.float32)
    idx, val = K.vq_sorted_gemm_batch_argmax(x.to(dev), sp, m["scale"].to(dev), cb0.to(dev), None, n)
    assert idx.shape == (B,) and val.shape == (B,)
    _, y64 = O.vq_gemv(x.numpy(), m["idx0"], None, cb0, None, m["scale"])
    _, y64r = O.vq_gemv(_fp16_scaled(x.numpy()), m["idx0"], None, cb0, None, m["scale"])
    for b in range(B):
        top = np.sort(y64r[b])[-2:]
        assert top[1] - top[0] > 1e-5 * abs(top[1]), b  # a unique winner at this seed
        assert int(idx[b]) == int(np.argmax(y64r[b])), b
        assert abs(float(val[b]) - y64r[b].max()) <= 1e-5 * abs(y64r[b].max()), b
        assert y64[b].max() - y64[b][int(idx[b])] <= TOL * np.abs(y64[b]).max(), b


def test_batch_argmax_ties_pick_lower_row(dev):
    """Two chunks with identical codes and scales (so the kernel sums their
    rows in the same order and the values tie exactly) hold the maximum of
    every activation row at rows 100 and 100 + 5 R: the lower row wins, as
    torch.argmax."""
    rows, n, B = 4096, 2048, 4
    m = synth.vq_matrix(9760, rows, n, bpw=2)
    i0 = m["idx0"].clone()
    R = K.SortedPlanes(i0, None, rows, n, device="cpu").rows_per_chunk
    sc = m["scale"].clone()
    i0[5 * R:6 * R] = i0[:R]
    sc[5 * R:6 * R] = sc[:R]
    cb = synth.codebook(9761)
    x = synth.activations(9762, (B, n), dtype=torch.float16)
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    x = x * torch.from_numpy(np.sign(y64[:, 100]).astype(np.float16))[:, None]
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    need = np.abs(y64).max() / (y64[:, 100] / float(sc[100])).min()
    sc[100] = sc[5 * R + 100] = float(2.0 ** np.ceil(np.log2(need) + 1))
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    assert np.all(np.argmax(y64, 1) == 100) and np.all(y64[:, 100] == y64[:, 5 * R + 100])
    sp = K.SortedPlanes(i0, None, rows, n, device=dev)
    (y,) = K.vq_sorted_gemm_batch(x.to(dev), [(sp, sc.to(dev))], cb.to(dev), None, n, slices=1)
    assert torch.equal(y[:, 100], y[:, 5 * R + 100])  # the tie is exact in the kernel too
    idx, val = K.vq_sorted_gemm_batch_argmax(x.to(dev), sp, sc.to(dev), cb.to(dev), None, n)
    assert idx.cpu().tolist() == [100] * B
    assert np.allclose(val.cpu().numpy(), y64[:, 100], rtol=1e-5)


def test_batch_gemm_errors(dev):
    m, cb0, _, sp = _mk(9770, 512, 2048, 2, dev)
    s = m["scale"].to(dev)
    with pytest.raises(Vq2Error, match="1..4 activation rows"):
        K.vq_sorted_gemm_batch(torch.zeros(5, 2048, device=dev), [(sp, s)], cb0.to(dev), None, 2048)
    # n = 65536: the fp16 activation of 2 rows alone is 256 KiB of LDS
    big = synth.vq_matrix(9771, 16, 65536, bpw=2)
    spb = K.SortedPlanes(big["idx0"], None, 16, 65536, device=dev)
    for B in (2, 4):
        with pytest.raises(Vq2Error, match="LDS"):
            K.vq_sorted_gemm_batch(torch.zeros(B, 65536, device=dev), [(spb, big["scale"].to(dev))], cb0.to(dev),
                                   None, 65536)


@pytest.mark.parametrize("B", [3, 4])
def test_batch_gemm_split_into_two_row_launches(dev, B):
    """4-row workgroups that would take more than half a CU's LDS run as
    launches of at most 2 rows: n = 32768 (4 rows: 256 KiB, 2 rows: 132
    KiB) and the LM head's 297-row chunks; logits and top-1 against the
    oracle on the activation as the kernel holds it."""
    from act_rounding import fp16_row_scaled

    cb = synth.codebook(9772)
    for rows, n, R in ((64, 32768, None), (700, 2048, 297)):
        m = synth.vq_matrix(9773 + n, rows, n, bpw=2)
        sp = K.SortedPlanes(m["idx0"], None, rows, n, device=dev, rows_per_chunk=R)
        x = synth.activations(9774 + B, (B, n), dtype=torch.float32) * 0.5
        (y,) = K.vq_sorted_gemm_batch(x.to(dev), [(sp, m["scale"].to(dev))], cb.to(dev), None, n)
        _, y64 = O.vq_gemv(fp16_row_scaled(x.numpy()), m["idx0"], None, cb, None, m["scale"])
        for b in range(B):
            assert O.max_rel_err(y.cpu().numpy()[b], y64[b]) < 1e-5, (n, b)
        idx, val = K.vq_sorted_gemm_batch_argmax(x.to(dev), sp, m["scale"].to(dev), cb.to(dev), None, n)
        assert idx.cpu().tolist() == [int(np.argmax(y64[b])) for b in range(B)], n


def test_batch_paths_graph_replays_match_eager(dev):
    """gate + up at batch 2 (one sorted batch launch, several slices per
    chunk summed in the launch) and the LM-head top-1 at batch 2, captured
    once; every replay, with eager work and synchronisations between the
    replays, equals the eager step bit for bit."""
    from compressai_amd.graph import DecodeStepGraph
    from compressai_amd.runtime import PackedLinear, PackedLMHead, PackedProjections

    n = 2048
    cbs = {"16": synth.codebook(9780).to(dev), "16_16": synth.codebook(9781).to(dev)}
    ms = [synth.vq_matrix(9782 + k, 6144, n, bpw=4) for k in range(2)]
    gu = PackedProjections([PackedLinear((6144, n), (16, 16), "mlp", [m["idx0"], m["idx1"]], m["scale"], cbs, dev)
                            for m in ms])
    mh = synth.vq_matrix(9784, 32768, n, bpw=2)
    head = PackedLMHead(PackedLinear((32768, n), (16,), "lm_head", [mh["idx0"]], mh["scale"], cbs, dev))
    assert K.sorted_batch_slices(gu.sorted, dev) > 1

    def step(x):
        g, u = gu(x, out_dtype=torch.float32)
        idx, val = head.argmax(x)
        return g, u, idx, val

    gstep = DecodeStepGraph(step, [synth.activations(9785, (2, n), dtype=torch.float16).to(dev)])
    for r in range(4):
        x = synth.activations(9786 + r, (2, n), dtype=torch.float16).to(dev)
        ref = [t.clone() for t in step(x)]
        torch.cuda.synchronize()
        out = [t.clone() for t in gstep(x)]
        torch.cuda.synchronize()
        for a, b in zip(out, ref):
            assert torch.equal(a, b), r


def test_batch4_split_graph_replays_match_eager(dev):
    """Logits and top-1 at batch 4 over 300-row chunks (4-row workgroups past
    80 KiB of LDS, so each call runs as two 2-row launches sharing one
    workspace) through a PackedLinear whose planes were released, captured
    once; every replay, with eager work and synchronisations between the
    replays, equals the eager step bit for bit."""
    from compressai_amd.graph import DecodeStepGraph
    from compressai_amd.runtime import PackedLinear, PackedLMHead

    n, rows = 2048, 4800
    cbs = {"16": synth.codebook(9790).to(dev)}
    mh = synth.vq_matrix(9791, rows, n, bpw=2)
    lin = PackedLinear((rows, n), (16,), "lm_head", [mh["idx0"]], mh["scale"], cbs, dev)
    lin.sorted = K.SortedPlanes(mh["idx0"], None, rows, n, device=dev, rows_per_chunk=300)
    lin.release_planes()
    head = PackedLMHead(lin)

    def step(x):
        y = lin(x, out_dtype=torch.float32)
        idx, val = head.argmax(x)
        return y, idx, val

    gstep = DecodeStepGraph(step, [synth.activations(9792, (4, n), dtype=torch.float16).to(dev)])
    for r in range(4):
        x = synth.activations(9793 + r, (4, n), dtype=torch.float16).to(dev)
        ref = [t.clone() for t in step(x)]
        torch.cuda.synchronize()
        out = [t.clone() for t in gstep(x)]
        torch.cuda.synchronize()
        for a, b in zip(out, ref):
            assert torch.equal(a, b), r
        assert ref[1].cpu().tolist() == ref[0].argmax(dim=1).cpu().tolist()
