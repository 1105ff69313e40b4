"""Containers of the reference (.vq2 with fixed-width streams, .vq2r) read
onto the device.  CPU tests: the safe loader, stream validation, the .vq2r
path and module construction.  GPU tests: the planes unpacked on the device
equal the codes that were packed, the .vq2r conversion round-trips, and the
modules built from a container compute what modules built from the planes
compute."""
import pickle

import numpy as np
import pytest
import torch

from compressai_amd import container as CT, synth
from compressai_amd import kernels as K
from vq2_containers import make_container

MATS = {
    "model.layers.0.self_attn.q_proj": ((96, 512), (16,), "layers.0.self_attn.q_proj"),
    "model.layers.0.mlp.gate_proj": ((64, 512), (16, 8), "layers.0.mlp.gate_proj"),
    "model.layers.0.mlp.down_proj": ((128, 256), (16, 16), "layers.0.mlp.down_proj"),
    "model.layers.1.self_attn.o_proj": ((72, 512), (16, 8), "layers.1.self_attn.o_proj"),
    "model.embed_tokens": ((200, 512), (16,), "embed_tokens"),
}


def _codebooks():
    cbs = {"16": synth.codebook(5000), "16_8": synth.codebook(5001, rows=256), "16_16": synth.codebook(5002)}
    return cbs, {"16": synth.codebook(5003)}


def _write(tmp_path, C, name="m.vq2"):
    path = tmp_path / name
    torch.save(C, path)
    return path


def test_safe_loader_reads_reference_layout_and_refuses_code(tmp_path):
    cbs, emb = _codebooks()
    C, _ = make_container(MATS, cbs, emb, seed=1)
    path = _write(tmp_path, C)
    D = CT.load_file(path)
    assert D["names"] == C["names"]
    assert isinstance(D["scales"]["model.embed_tokens"], np.ndarray)
    assert np.array_equal(D["streams"]["16"]["counts"], C["streams"]["16"]["counts"])
    # a pickle that would call something is refused by the loader
    bad = tmp_path / "bad.vq2"
    torch.save({"names": [], "meta": {}, "x": print}, bad)
    with pytest.raises(pickle.UnpicklingError, match="Weights only"):
        CT.load_file(bad)


def test_stream_validation_before_upload(tmp_path):
    cbs, emb = _codebooks()
    C, _ = make_container(MATS, cbs, emb, seed=2)
    C["streams"]["16_16"] = dict(C["streams"]["16_16"], mode="ans", ans=torch.zeros(4, dtype=torch.uint32))
    with pytest.raises(K.Vq2Error, match="ANS"):
        CT.decode_indices(C, "cpu")
    C, _ = make_container(MATS, cbs, emb, seed=2)
    C["streams"]["16_8"]["sizes"] = C["streams"]["16_8"]["sizes"][:1]
    with pytest.raises(K.Vq2Error, match="sizes"):
        CT.decode_indices(C, "cpu")
    C, _ = make_container(MATS, cbs, emb, seed=2)
    with pytest.raises(K.Vq2Error, match="GPU"):
        CT.decode_indices(C, "cpu")


def test_vq2r_read_and_modules_on_cpu(tmp_path):
    """A .vq2r (decoded planes) needs no unpacking: it reads on the CPU and
    the modules get the planes, cfgs and codebooks the container names."""
    cbs, emb = _codebooks()
    C, planes = make_container(MATS, cbs, emb, seed=3)
    idx = {nm: [torch.from_numpy(p.astype(np.uint8) if b <= 8 else p.astype(np.uint16).view(np.int16))
                for p, b in zip(planes[nm], MATS[nm][1])] for nm in MATS}
    R = dict(format="vq2r", names=C["names"], meta=C["meta"], idx=idx,
             scales={nm: torch.from_numpy(s) for nm, s in C["scales"].items()}, codebooks=C["codebooks"],
             codebooks_embed=C["codebooks_embed"], dense=C["dense"])
    path = _write(tmp_path, R, "m.vq2r")
    got = CT.read_container(path, "cpu")
    for nm in MATS:
        for a, b in zip(got["idx"][nm], idx[nm]):
            assert a.dtype == b.dtype and torch.equal(a, b)
    mods = CT.load_packed_linears(got, "cpu")
    g = mods["model.layers.0.mlp.gate_proj"]
    assert g.cfg == (16, 8) and g.idx1.dtype == torch.uint8 and g._planes()[3].shape == (256, 8)
    assert mods["lm_head"].lin is mods["model.embed_tokens"]
    assert torch.equal(mods["model.embed_tokens"]._planes()[2].float(), emb["16"].half().bfloat16().float())
    assert "lm_head" not in CT.load_packed_linears(got, "cpu", tie_embeddings=False)


@pytest.mark.gpu
def test_decode_on_gpu_matches_packed_codes(dev, tmp_path):
    cbs, emb = _codebooks()
    C, planes = make_container(MATS, cbs, emb, seed=4)
    R = CT.read_container(_write(tmp_path, C), dev)
    for nm, (_, cfg, _) in MATS.items():
        for p, b, got in zip(planes[nm], cfg, R["idx"][nm]):
            assert got.is_cuda and got.shape == p.shape
            if b <= 8:
                assert got.dtype == torch.uint8
                assert np.array_equal(got.cpu().numpy().astype(np.int64), p)
            else:
                assert got.dtype == torch.int16
                assert np.array_equal(got.cpu().numpy().view(np.uint16).astype(np.int64), p)


@pytest.mark.gpu
def test_convert_to_runtime_round_trip_and_modules(dev, tmp_path):
    """.vq2 -> .vq2r (decoded once on the GPU) reads back to the same planes,
    and every module built from the container equals one built from the
    planes directly, bit for bit, at batch 1 and 5."""
    from compressai_amd.runtime import PackedLinear

    cbs, emb = _codebooks()
    C, planes = make_container(MATS, cbs, emb, seed=5)
    src = _write(tmp_path, C)
    dst = tmp_path / "m.vq2r"
    CT.convert_to_runtime(src, dst, dev)
    R1 = CT.read_container(src, dev)
    R2 = CT.read_container(dst, dev)
    for nm in MATS:
        for a, b in zip(R1["idx"][nm], R2["idx"][nm]):
            assert torch.equal(a, b)
    mods = CT.load_packed_linears(R2, dev, cb_dtype=torch.float16)
    for nm, (shape, cfg, tag) in MATS.items():
        pl = [torch.from_numpy(p.astype(np.uint8) if b <= 8 else p.astype(np.uint16).view(np.int16))
              for p, b in zip(planes[nm], cfg)]
        cb = {k: v.to(dev) for k, v in (emb if nm.endswith("embed_tokens") else cbs).items()}
        ref = PackedLinear(shape, cfg, tag, pl, torch.from_numpy(C["scales"][nm]), cb, dev)
        for B in (1, 5):
            x = synth.activations(5100 + B, (B, shape[1])).to(dev)
            assert torch.equal(mods[nm](x, out_dtype=torch.float32), ref(x, out_dtype=torch.float32)), (nm, B)
    x = synth.activations(5110, (1, 512)).to(dev)
    i, _ = mods["lm_head"].argmax(x)
    assert int(i[0]) == int(torch.argmax(mods["model.embed_tokens"](x, out_dtype=torch.float32)[0]))
