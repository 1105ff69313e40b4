"""GPU parity of the code-sorted VQ GEMV (vq2_sorted_gemv / _argmax, through
the C ABI) against the fp64 oracle on the same seeded inputs: the config 1-3
shapes, ragged row counts and non-power-of-two widths, 2, 3 (16,8) and 4 bpw, fp16 and
bf16 codebooks, the fused RHT prologue and pre-rotated activations, one or
several workgroups per chunk, several matrices per launch, and the fused
LM-head top-1 (ties resolve to the lower row, as torch.argmax).

Tolerance: max_i |y_i - ref_i| / max_i |ref_i| <= 1e-3 (the decode-path
contract), observed ~1e-7: fp32 accumulation in another order."""
import numpy as np
import pytest
import torch

from compressai_amd import kernels as K, synth
from oracle import vq2_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _mk(seed, rows, n, bpw, dev, cb_dtype=torch.float16):
    m = synth.vq_matrix(seed, rows, n, bpw=bpw)
    cb0 = synth.codebook(seed + 1, dtype=cb_dtype)
    cb1 = synth.codebook(seed + 2, 256 if bpw == 3 else 65536, dtype=cb_dtype) if bpw > 2 else None
    sp = K.SortedPlanes(m["idx0"], m["idx1"], rows, n, device=dev)
    return m, cb0, cb1, sp


@pytest.mark.parametrize("rows,n,bpw,fused,slices", [
    (2048, 2048, 2, True, None),     # configs[0] / o projection
    (6144, 2048, 4, True, None),     # gate / up
    (2048, 6144, 4, True, None),     # down, 3 x 2048-point RHT blocks
    (1000, 512, 2, False, 3),
    (97, 800, 2, False, 1),          # ng = 100: not a power of two
    (517, 2048, 4, True, 7),
    (300, 2048, 2, True, 64),        # more slices than iterations per chunk
    (2048, 2048, 3, True, None),     # (16,8): stage-2 uint8 codes into the 256-row codebook
    (512, 6144, 3, True, None),
    (97, 800, 3, False, 2),
])
def test_sorted_gemv_vs_oracle(dev, rows, n, bpw, fused, slices):
    m, cb0, cb1, sp = _mk(9500 + rows + n, rows, n, bpw, dev)
    x = synth.activations(9501 + rows, n, dtype=torch.float16)
    perm, sign = synth.permutation(9502, n), synth.signs(9503, n)
    if fused:
        (y,) = K.vq_sorted_gemv(x.to(dev), [(sp, m["scale"].to(dev))], cb0.to(dev), None if cb1 is None else cb1.to(dev),
                                n, perm.to(dev), sign.to(dev), 2048, slices=slices)
        xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    else:
        xr = (synth.activations(9504 + rows, n, dtype=torch.float32) * 0.5).numpy()
        (y,) = K.vq_sorted_gemv(torch.from_numpy(xr).to(dev), [(sp, m["scale"].to(dev))], cb0.to(dev),
                                None if cb1 is None else cb1.to(dev), n, hb=0, slices=slices)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert y.shape == (rows,)
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL


@pytest.mark.parametrize("rows,n,bpw,R,slices", [
    (700, 2048, 2, 350, None),    # 17-bit positions: bit 16 in each field's high byte
    (1200, 2048, 4, 300, 3),
    (300, 6144, 4, 120, 2),       # 6144 wide: 10 group bits + 7 row bits
    (600, 2048, 3, 511, None),    # (16,8), the tallest chunk
])
def test_sorted_taller_chunks_vs_oracle(dev, rows, n, bpw, R, slices):
    """Chunks of up to 511 rows (the LM head's default, 297 rows, is one of
    them): the batch-1 kernel with the RHT prologue (row sums of 256 rows
    or more in two halves), the batch kernel at B = 2 and 4 and, at 2 bpw,
    the fused top-1 of both, against the oracle."""
    from act_rounding import fp16_row_scaled

    m = synth.vq_matrix(9560 + R, rows, n, bpw=bpw)
    cb0 = synth.codebook(9561)
    cb1 = synth.codebook(9562, 256 if bpw == 3 else 65536) if bpw > 2 else None
    sp = K.SortedPlanes(m["idx0"], m["idx1"], rows, n, device=dev, rows_per_chunk=R)
    assert sp.rows_per_chunk == R
    c0, c1, sc = cb0.to(dev), None if cb1 is None else cb1.to(dev), m["scale"].to(dev)
    x = synth.activations(9563, n, dtype=torch.float16)
    perm, sign = synth.permutation(9564, n), synth.signs(9565, n)
    (y,) = K.vq_sorted_gemv(x.to(dev), [(sp, sc)], c0, c1, n, perm.to(dev), sign.to(dev), 2048, slices=slices)
    xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL
    for B in (2, 4):
        xb = synth.activations(9566 + B, (B, n), dtype=torch.float32) * 0.5
        (yb,) = K.vq_sorted_gemm_batch(xb.to(dev), [(sp, sc)], c0, c1, n, slices=slices)
        # the batch kernel's fp16 activation with a power-of-two scale per row
        _, yb64 = O.vq_gemv(fp16_row_scaled(xb.numpy()), m["idx0"], m["idx1"], cb0, cb1, m["scale"])
        for b in range(B):
            assert O.max_rel_err(yb.cpu().numpy()[b], yb64[b]) < 1e-5, (B, b)
        if bpw == 2:
            idx, val = K.vq_sorted_gemm_batch_argmax(xb.to(dev), sp, sc, c0, None, n)
            for b in range(B):
                assert int(idx[b]) == int(np.argmax(yb64[b])), (B, b)
    if bpw == 2:
        idx, val = K.vq_sorted_gemv_argmax(x.to(dev), sp, sc, c0, None, n, perm.to(dev), sign.to(dev), 2048)
        assert int(idx[0]) == int(np.argmax(y64[0]))
        assert abs(float(val[0]) - y64[0].max()) <= 1e-5 * abs(y64[0].max())


@pytest.mark.parametrize("bpw", [2, 4])
def test_sorted_mixed_lane_groups_in_one_launch(dev, bpw):
    """One launch over matrices whose chunks take four 16-lane accumulator
    groups (11 and 32 rows), two 32-lane groups (40 rows) and the
    taller-chunk path (300 rows): the batch-1 kernel with the RHT prologue at
    one slice and three, and the batch kernel at B = 4, against the oracle."""
    from act_rounding import fp16_row_scaled

    n = 2048
    shapes = ((500, 11), (300, 32), (260, 40), (700, 300))
    ms = [synth.vq_matrix(9580 + k, rows, n, bpw=bpw) for k, (rows, _) in enumerate(shapes)]
    cb0 = synth.codebook(9585)
    cb1 = synth.codebook(9586) if bpw == 4 else None
    sps = [K.SortedPlanes(m["idx0"], m["idx1"], rows, n, device=dev, rows_per_chunk=R)
           for m, (rows, R) in zip(ms, shapes)]
    assert [sp.rows_per_chunk for sp in sps] == [R for _, R in shapes]
    c0, c1 = cb0.to(dev), None if cb1 is None else cb1.to(dev)
    mats = [(sp, m["scale"].to(dev)) for sp, m in zip(sps, ms)]
    x = synth.activations(9587, n, dtype=torch.float16)
    perm, sign = synth.permutation(9588, n), synth.signs(9589, n)
    xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    for slices in (1, 3):
        ys = K.vq_sorted_gemv(x.to(dev), mats, c0, c1, n, perm.to(dev), sign.to(dev), 2048, slices=slices)
        for k, m in enumerate(ms):
            _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
            assert O.max_rel_err(ys[k].cpu().numpy(), y64[0]) < TOL, (slices, k)
    xb = synth.activations(9590, (4, n), dtype=torch.float32) * 0.5
    ybs = K.vq_sorted_gemm_batch(xb.to(dev), mats, c0, c1, n)
    xk = fp16_row_scaled(xb.numpy())
    for k, m in enumerate(ms):
        _, yb64 = O.vq_gemv(xk, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
        for b in range(4):
            assert O.max_rel_err(ybs[k].cpu().numpy()[b], yb64[b]) < 1e-5, (k, b)


def test_sorted_gemv_bf16_codebook_and_outputs(dev):
    rows, n = 1536, 2048
    m, cb0, cb1, sp = _mk(9520, rows, n, 4, dev, cb_dtype=torch.bfloat16)
    x = synth.activations(9521, n, dtype=torch.bfloat16)
    sc = m["scale"].to(torch.bfloat16)
    perm, sign = synth.permutation(9522, n), synth.signs(9523, n)
    (y,) = K.vq_sorted_gemv(x.to(dev), [(sp, sc.to(dev))], cb0.to(dev), cb1.to(dev), n, perm.to(dev), sign.to(dev),
                            2048, out_dtype=torch.bfloat16)
    xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, sc)
    err = np.abs(y.float().cpu().numpy() - y64[0])
    assert np.all(err <= 2.0 ** -8 * np.abs(y64[0]) + 1e-5 * np.abs(y64[0]).max())  # one bf16 rounding


def test_sorted_gemv_qkv_segments_and_determinism(dev):
    """q / k / v in one launch (shared RHT), equal to the oracle and to
    itself bit for bit over repeated calls."""
    n = 2048
    cb0 = synth.codebook(9530)
    shapes = [2048, 512, 512]
    ms = [synth.vq_matrix(9531 + k, r, n, bpw=2) for k, r in enumerate(shapes)]
    sps = [K.SortedPlanes(m["idx0"], None, r, n, device=dev) for m, r in zip(ms, shapes)]
    x = synth.activations(9535, n, dtype=torch.float16)
    perm, sign = synth.permutation(9536, n), synth.signs(9537, n)
    mats = [(sp, m["scale"].to(dev)) for sp, m in zip(sps, ms)]
    ys = K.vq_sorted_gemv(x.to(dev), mats, cb0.to(dev), None, n, perm.to(dev), sign.to(dev), 2048)
    xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    for y, m in zip(ys, ms):
        _, y64 = O.vq_gemv(xr, m["idx0"], None, cb0, None, m["scale"])
        assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL
    again = K.vq_sorted_gemv(x.to(dev), mats, cb0.to(dev), None, n, perm.to(dev), sign.to(dev), 2048)
    for a, b in zip(ys, again):
        assert torch.equal(a, b)


def _sorted_counters(dev):
    """The arrival-counter header of this stream's sorted workspace."""
    ws = K._WS[(dev.index, torch.cuda.current_stream(dev).cuda_stream, True)]
    return ws[:16384].view(torch.int32)


@pytest.mark.parametrize("rows,n,bpw,slices,n_mat", [
    (6144, 2048, 4, 5, 2),    # the gate + up call
    (2048, 6144, 4, 7, 1),    # down
    (700, 1024, 2, 33, 3),    # many slices, several matrices
])
def test_sorted_in_kernel_reduce_fresh_inputs(dev, rows, n, bpw, slices, n_mat):
    """The chunk's last workgroup sums the slices inside the launch.  Twelve
    launches back to back on one stream, each with another activation and no
    synchronisation in between: a share read before its writer's store
    landed (or left from the previous launch) would show as an error far
    above the tolerance.  Every output matches the gather kernel on the same
    input to accumulation-order rounding, and the counters end at zero."""
    cb0 = synth.codebook(9580).to(dev)
    cb1 = synth.codebook(9581).to(dev) if bpw == 4 else None
    ms = [synth.vq_matrix(9582 + k, rows, n, bpw=bpw) for k in range(n_mat)]
    sps = [K.SortedPlanes(m["idx0"], m["idx1"], rows, n, device=dev) for m in ms]
    mats = [(sp, m["scale"].to(dev)) for sp, m in zip(sps, ms)]
    perm, sign = synth.permutation(9586, n).to(dev), synth.signs(9587, n).to(dev)
    xs = [synth.activations(9600 + i, n, dtype=torch.float16).to(dev) for i in range(12)]
    hb = min(2048, n)
    outs = [K.vq_sorted_gemv(x, mats, cb0, cb1, n, perm, sign, hb, slices=slices) for x in xs]
    torch.cuda.synchronize(dev)
    assert int(_sorted_counters(dev).abs().sum()) == 0
    for i, x in enumerate(xs):
        for k, m in enumerate(ms):
            (yg,) = K.vq_gemv_rht(x, [(m["idx0"].to(dev), None if m["idx1"] is None else m["idx1"].to(dev),
                                       m["scale"].to(dev), rows)], cb0, cb1, n, perm, sign, hb)
            assert O.max_rel_err(outs[i][k].cpu().numpy(), yg.cpu().numpy()) < 1e-5, (i, k)


def test_sorted_multi_slice_graph_replays(dev):
    """A multi-slice launch (partials in the workspace, summed by the chunk's
    last workgroup) captured in a HIP graph: every replay, with eager launches
    on the same matrix in between, equals the eager result bit for bit."""
    rows, n = 6144, 2048
    m, cb0, cb1, sp = _mk(9570, rows, n, 4, dev)
    x = synth.activations(9571, n, dtype=torch.float16).to(dev)
    perm, sign = synth.permutation(9572, n).to(dev), synth.signs(9573, n).to(dev)
    sc, c0, c1 = m["scale"].to(dev), cb0.to(dev), cb1.to(dev)
    y = torch.empty(rows, device=dev)
    run = lambda: K.vq_sorted_gemv(x, [(sp, sc)], c0, c1, n, perm, sign, 2048, ys=[y], slices=5)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        run()
        ref = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run()
    torch.cuda.synchronize(dev)
    for r in range(4):
        y.zero_()
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(y, ref), r
        run()                                   # eager call between replays
        torch.cuda.synchronize(dev)
        assert torch.equal(y, ref), r
    xr = O.rht(x.cpu(), perm.cpu(), sign.cpu(), 2048).astype(np.float32)
    _, y64 = O.vq_gemv(xr, m["idx0"], m["idx1"], cb0, cb1, m["scale"])
    assert O.max_rel_err(ref.cpu().numpy(), y64[0]) < TOL


def test_sorted_matches_gather_kernel(dev):
    """The sorted kernel and the gather kernel (vq_gemv_rht) agree to fp32
    accumulation-order rounding on the gate/up shape."""
    rows, n = 6144, 2048
    m, cb0, cb1, sp = _mk(9540, rows, n, 4, dev)
    x = synth.activations(9541, n, dtype=torch.float16).to(dev)
    perm, sign = synth.permutation(9542, n).to(dev), synth.signs(9543, n).to(dev)
    (ys,) = K.vq_sorted_gemv(x, [(sp, m["scale"].to(dev))], cb0.to(dev), cb1.to(dev), n, perm, sign, 2048)
    (yg,) = K.vq_gemv_rht(x, [(m["idx0"].to(dev), m["idx1"].to(dev), m["scale"].to(dev), rows)], cb0.to(dev),
                          cb1.to(dev), n, perm, sign, 2048)
    assert O.max_rel_err(ys.cpu().numpy(), yg.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("fused", [False, True])
def test_sorted_lm_head_top1_full_size(dev, fused):
    """configs[2] LM head 151936 x 2048 at 2 bpw, batch 1: the fused top-1
    equals the argmax of the oracle's logits."""
    rows, n = 151936, 2048
    m, cb0, _, sp = _mk(9550, rows, n, 2, dev)
    if 2 * 255 * K._cu_count(dev) < rows:  # the tall-matrix chunking: 17-bit positions
        assert sp.rows_per_chunk > 255 and sp.n_chunks % (2 * K._cu_count(dev)) == 0
    perm, sign = synth.permutation(9552, n), synth.signs(9553, n)
    if fused:
        x = synth.activations(9551, n, dtype=torch.float16)
        idx, val = K.vq_sorted_gemv_argmax(x.to(dev), sp, m["scale"].to(dev), cb0.to(dev), None, n, perm.to(dev),
                                           sign.to(dev), 2048)
        xr = O.rht(x, perm, sign, 2048).astype(np.float32)
    else:
        xr = synth.activations(9554, n, dtype=torch.float32).numpy()
        idx, val = K.vq_sorted_gemv_argmax(torch.from_numpy(xr).to(dev), sp, m["scale"].to(dev), cb0.to(dev), None,
                                           n)
    _, y64 = O.vq_gemv(xr, m["idx0"], None, cb0, None, m["scale"])
    top = np.sort(y64[0])[-2:]
    assert top[1] - top[0] > 1e-5 * abs(top[1])  # a unique winner at this seed
    assert int(idx[0]) == int(np.argmax(y64[0]))
    assert abs(float(val[0]) - y64[0].max()) <= 1e-5 * abs(y64[0].max())


def test_sorted_top1_ties_pick_lower_row(dev):
    """Two chunks with identical codes and scales (so the kernel sums their
    rows in the same order and the values tie exactly) hold the maximum at
    rows 100 and 100 + 5 R: the lower row wins, as torch.argmax."""
    rows, n = 4096, 2048
    m = synth.vq_matrix(9560, rows, n, bpw=2)
    i0 = m["idx0"].clone()
    R = K.SortedPlanes(i0, None, rows, n, device="cpu").rows_per_chunk
    sc = m["scale"].clone()
    i0[5 * R:6 * R] = i0[:R]
    sc[5 * R:6 * R] = sc[:R]
    cb = synth.codebook(9561)
    x = synth.activations(9562, n, dtype=torch.float32)
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    if y64[0, 100] < 0:
        x = -x
        _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    boost = float(2.0 ** np.ceil(np.log2(np.abs(y64).max() / (y64[0, 100] / float(sc[100])) + 1)))
    sc[100] = sc[5 * R + 100] = boost
    _, y64 = O.vq_gemv(x, i0, None, cb, None, sc)
    assert np.argmax(y64[0]) == 100 and y64[0, 100] == y64[0, 5 * R + 100]
    sp = K.SortedPlanes(i0, None, rows, n, device=dev)
    (y,) = K.vq_sorted_gemv(x.to(dev), [(sp, sc.to(dev))], cb.to(dev), None, n, hb=0, slices=1)
    assert float(y[100]) == float(y[5 * R + 100])   # the tie is exact in the kernel too
    idx, _ = K.vq_sorted_gemv_argmax(x.to(dev), sp, sc.to(dev), cb.to(dev), None, n)
    assert int(idx[0]) == 100


def test_sorted_gemv_16_8_bf16_and_batch_kernel(dev):
    """(16,8) on the sorted layout with bf16 codebooks and scales, through
    the batch-1 kernel and the batch 2 / 4 kernel, against the oracle (the
    batch kernel rounds the activation to fp16 under a power-of-two row
    scale: tested against the oracle fed that rounded activation)."""
    from act_rounding import fp16_row_scaled

    rows, n = 1024, 2048
    m, cb0, cb1, sp = _mk(9560, rows, n, 3, dev, cb_dtype=torch.bfloat16)
    assert sp.s2_kind == 2
    sc = m["scale"].to(torch.bfloat16)
    xr = synth.activations(9561, (4, n), dtype=torch.float32)
    (y,) = K.vq_sorted_gemv(xr[0].to(dev), [(sp, sc.to(dev))], cb0.to(dev), cb1.to(dev), n, hb=0)
    _, y64 = O.vq_gemv(xr[:1].numpy(), m["idx0"], m["idx1"], cb0, cb1, sc)
    assert O.max_rel_err(y.cpu().numpy(), y64[0]) < TOL
    for B in (2, 4):
        (yb,) = K.vq_sorted_gemm_batch(xr[:B].to(dev), [(sp, sc.to(dev))], cb0.to(dev), cb1.to(dev), n)
        _, yr = O.vq_gemv(fp16_row_scaled(xr[:B].numpy()), m["idx0"], m["idx1"], cb0, cb1, sc)
        assert max(O.max_rel_err(yb[b].cpu().numpy(), yr[b]) for b in range(B)) < 1e-5


def test_sorted_16_8_refuses_a_65536_row_stage2_mismatch(dev):
    """A (16,8) sorted matrix needs the [256, 8] stage-2 codebook of cb0's
    dtype; a (16,16) one a [65536, 8]; one launch takes one kind."""
    m, cb0, cb1, sp = _mk(9570, 64, 512, 3, dev)
    x = synth.activations(9571, 512, dtype=torch.float32).to(dev)
    with pytest.raises(K.Vq2Error):
        K.vq_sorted_gemv(x, [(sp, m["scale"].to(dev))], cb0.to(dev), None, 512, hb=0)
    m4, _, c4, sp4 = _mk(9572, 64, 512, 4, dev)
    with pytest.raises(K.Vq2Error):
        K.vq_sorted_gemv(x, [(sp, m["scale"].to(dev)), (sp4, m4["scale"].to(dev))], cb0.to(dev), c4.to(dev), 512,
                         hb=0)
