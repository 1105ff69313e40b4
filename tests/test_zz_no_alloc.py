"""vq2_gemm_small_m_noalloc (the entry point that allocates nothing) against
vq2_gemm_small_m with a caller workspace, through the C ABI: bit-identical
outputs on two calls in a row, the second smaller, and a shape whose
split-K partials exceed the library's scratch is refused without a launch."""
import numpy as np
import pytest
import torch

from compressai_amd import _lib, synth
from oracle import vq2_oracle as O

pytestmark = pytest.mark.gpu


def _args(x, m, cb0, cb1, out, n, y):
    i1 = m["idx1"]
    s2 = _lib.S2_NONE if i1 is None else (_lib.S2_U8 if i1.dtype == torch.uint8 else _lib.S2_U16)
    return [x.data_ptr(), _lib.DT_F16, x.shape[0], n, m["idx0"].data_ptr(), None if i1 is None else i1.data_ptr(),
            s2, cb0.data_ptr(), None if cb1 is None else cb1.data_ptr(), _lib.DT_F16, m["scale"].data_ptr(),
            _lib.DT_F16, y.data_ptr(), _lib.DT_F32, out, out, n, 1.0]


def _on(dev, m):
    return {k: (None if v is None else v.to(dev)) for k, v in m.items()}


def test_noalloc_matches_workspace_entry(dev):
    L = _lib.load()
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    cb0 = synth.codebook(9700).to(dev)
    cb1 = synth.codebook(9701).to(dev)
    cases = [(64, 6144, 2048, 4), (5, 512, 2048, 2)]  # the second call is smaller
    for i, (M, out, n, bpw) in enumerate(cases):
        m = _on(dev, synth.vq_matrix(9702 + i, out, n, bpw=bpw))
        c1 = cb1 if bpw == 4 else None
        x = synth.activations(9710 + i, (M, n), dtype=torch.float16).to(dev)
        need = int(L.vq2_gemm_small_m_workspace(M, out, n))
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES, (need, M, out, n)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        y_ref = torch.full((M, out), float("nan"), dtype=torch.float32, device=dev)
        y = torch.full((M, out), float("nan"), dtype=torch.float32, device=dev)
        _lib.check(L.vq2_gemm_small_m(*_args(x, m, cb0, c1, out, n, y_ref), ws.data_ptr(), need, stream))
        _lib.check(L.vq2_gemm_small_m_noalloc(*_args(x, m, cb0, c1, out, n, y), stream), "noalloc")
        torch.cuda.synchronize(dev)
        assert torch.equal(y, y_ref), (M, out, n)
        _, y64 = O.vq_gemv(x.cpu(), m["idx0"].cpu(), None if m["idx1"] is None else m["idx1"].cpu(), cb0.cpu(),
                           None if c1 is None else c1.cpu(), m["scale"].cpu())
        yh = y.cpu().numpy()
        assert max(O.max_rel_err(yh[b], y64[b]) for b in range(M)) < 1e-3


def test_noalloc_refuses_shapes_beyond_its_scratch(dev):
    L = _lib.load()
    torch.cuda.set_device(dev)
    M, out, n = 64, 151936, 2048
    need = int(L.vq2_gemm_small_m_workspace(M, out, n))
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    cb0 = synth.codebook(9720).to(dev)
    i0 = torch.zeros((out, n // 8), dtype=torch.int16, device=dev)
    sc = torch.ones(out, dtype=torch.float16, device=dev)
    x = torch.zeros((M, n), dtype=torch.float16, device=dev)
    y = torch.full((M, out), 7.0, dtype=torch.float32, device=dev)
    st = L.vq2_gemm_small_m_noalloc(x.data_ptr(), _lib.DT_F16, M, n, i0.data_ptr(), None, _lib.S2_NONE,
                                    cb0.data_ptr(), None, _lib.DT_F16, sc.data_ptr(), _lib.DT_F16, y.data_ptr(),
                                    _lib.DT_F32, out, out, n, 1.0, torch.cuda.current_stream(dev).cuda_stream)
    assert st == _lib.ERR_UNSUPPORTED
    assert "scratch" in L.vq2_last_error().decode()
    torch.cuda.synchronize(dev)
    assert bool((y == 7.0).all())  # nothing was launched
