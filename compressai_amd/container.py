"""Compressed-model containers of the reference, read onto the device.

A ``.vq2`` container is a ``torch.save`` dict (vq2/export.py:88-118):
``names``, ``meta[name] = {shape, cfg, tag}``, ``scales[name]``,
``codebooks`` / ``codebooks_embed`` (keyed by stage key) and ``dense``, plus
one index *stream* per stage key ``"_".join(cfg[:i+1])`` ("16", "16_8",
"16_16", ...).  A stream holds the stage-i codes of every matrix whose cfg
has that key, concatenated in ``names`` order (``sizes`` gives each one's
count), either fixed-width packed (``mode "fixed"``: little-endian bit
stream, ``bits`` = the key's last field, vq2/export.py:39-70) or ANS coded
(``mode "ans"``).  A ``.vq2r`` container is the same dict with the streams
already decoded into ``idx[name] = [plane per stage]`` (vq2/runtime.py:
154-199).

``read_container`` follows vq2/runtime.py:184-199, except that a fixed-width
stream is uploaded once and unpacked on the GPU (``vq2_unpack_fixed``)
straight into the int16 code planes the kernels read; the planes of 8-bit
stages become uint8 on the device, as the reference's ``decode_indices``
gives them.  ANS streams need the reference's entropy coder (the third-party
``constriction`` package), which this build does not include: they are
refused with an error that names the remedy (``convert_to_runtime`` where the
coder is installed, vq2/runtime.py:202-206).

Files are loaded with ``torch.load(weights_only=True)``; a reference-written
``.vq2`` holds numpy arrays (scales, symbol counts), so numpy's array
reconstructors are allowed, nothing else.
"""
from __future__ import annotations

import numpy as np
import torch

from . import kernels as K
from .runtime import PackedLinear, PackedLMHead, cfg_key


def _numpy_safe_globals():
    from numpy._core.multiarray import _reconstruct

    safe = [_reconstruct, (_reconstruct, "numpy.core.multiarray._reconstruct"), np.ndarray, np.dtype]
    for t in (np.bool_, np.uint8, np.int8, np.uint16, np.int16, np.uint32, np.int32, np.uint64, np.int64,
              np.float16, np.float32, np.float64):
        safe.append(type(np.dtype(t)))
    return safe


def load_file(path) -> dict:
    """The container dict of a ``.vq2`` / ``.vq2r`` file (safe loader)."""
    with torch.serialization.safe_globals(_numpy_safe_globals()):
        C = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(C, dict) or "names" not in C or "meta" not in C:
        raise K.Vq2Error(f"{path}: not a vq2 container")
    return C


def _owners(C, key):
    """Matrices whose cfg has stage key `key`, in stream order, with the stage index."""
    out = []
    for nm in C["names"]:
        cfg = C["meta"][nm]["cfg"]
        keys = [cfg_key(cfg, j) for j in range(len(cfg))]
        if key in keys:
            out.append((nm, keys.index(key)))
    return out


def _as_tensor(a):
    return a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))


def _check_streams(C):
    """(key, bits, sizes, owners) of every stream; refuses what cannot be
    unpacked here before anything is uploaded."""
    out = []
    for key, e in C["streams"].items():
        bits = int(e["bits"])
        sizes = [int(s) for s in e["sizes"]]
        if e["mode"] == "ans":
            raise K.Vq2Error(f"stream {key} is ANS coded: decode it where the constriction coder is installed "
                             "(vq2.runtime.convert_to_runtime writes a .vq2r) and load that file")
        if e["mode"] != "fixed":
            raise K.Vq2Error(f"stream {key}: unknown mode {e['mode']!r}")
        if bits not in (4, 8, 12, 16):
            raise K.Vq2Error(f"stream {key}: {bits}-bit symbols (the packings are 4, 8, 12 and 16 bits)")
        owners = _owners(C, key)
        if len(owners) != len(sizes):
            raise K.Vq2Error(f"stream {key}: {len(sizes)} sizes for {len(owners)} matrices")
        for (nm, _), sz in zip(owners, sizes):
            rows = int(C["meta"][nm]["shape"][0])
            if sz % rows:
                raise K.Vq2Error(f"stream {key}: {sz} codes of {nm} do not fill {rows} rows")
        out.append((key, bits, sizes, owners))
    return out


def decode_indices(C, device) -> dict:
    """{name: [code plane per stage]} on `device` from the container's
    streams (vq2/runtime.py:154-181): int16 planes for stages over 8 bits
    (uint16 codes), uint8 planes for stages of 8 bits or fewer."""
    streams = _check_streams(C)
    device = torch.device(device)
    if device.type != "cuda":
        raise K.Vq2Error("decode_indices unpacks on the GPU: give a cuda device")
    idx = {nm: [None] * len(C["meta"][nm]["cfg"]) for nm in C["names"]}
    for key, bits, sizes, owners in streams:
        buf = _as_tensor(C["streams"][key]["fixed"]).reshape(-1).view(torch.uint8).to(device)
        codes = K.vq_unpack_fixed(buf, bits, sum(sizes))
        off = 0
        for (nm, i), sz in zip(owners, sizes):
            rows = int(C["meta"][nm]["shape"][0])
            plane = codes[off:off + sz].view(rows, -1)
            idx[nm][i] = plane.to(torch.uint8) if bits <= 8 else plane.clone()
            off += sz
        del codes, buf
    return idx


def read_container(path, device) -> dict:
    """``.vq2`` or ``.vq2r`` -> the runtime dict of vq2/runtime.py:184-199
    (format "vq2r"), with the index planes on `device`."""
    C = load_file(path)
    device = torch.device(device)
    if C.get("format") == "vq2r":
        idx = {nm: [_as_tensor(p).to(device) for p in planes] for nm, planes in C["idx"].items()}
    else:
        idx = decode_indices(C, device)
    scales = {nm: _as_tensor(s) for nm, s in C["scales"].items()}
    return dict(format="vq2r", names=C["names"], meta=C["meta"], idx=idx, scales=scales,
                codebooks=C["codebooks"], codebooks_embed=C.get("codebooks_embed", {}), dense=C.get("dense", {}))


def convert_to_runtime(src, dst, device) -> None:
    """Decode a fixed-width ``.vq2`` once (on the GPU) and save the ``.vq2r``
    runtime form with CPU planes (vq2/runtime.py:202-206)."""
    R = read_container(src, device)
    R["idx"] = {nm: [p.cpu() for p in planes] for nm, planes in R["idx"].items()}
    torch.save(R, dst)


def load_packed_linears(R, device, cb_dtype=torch.bfloat16, tie_embeddings: bool = True) -> dict:
    """{name: PackedLinear} of a runtime dict (the quantized-module part of
    vq2/runtime.py:load_packed, 209-242): codebooks cast to `cb_dtype` (the
    reference uses bf16), the embedding matrix on ``codebooks_embed``, and
    ``"lm_head"`` a PackedLMHead over the embedding's weights when
    `tie_embeddings` (the model config's ``tie_word_embeddings``)."""
    device = torch.device(device)
    cb_lin = {k: _as_tensor(v).to(device=device, dtype=cb_dtype) for k, v in R["codebooks"].items()}
    cb_emb = {k: _as_tensor(v).to(device=device, dtype=cb_dtype) for k, v in R.get("codebooks_embed", {}).items()}
    mods, emb = {}, None
    for nm in R["names"]:
        m = R["meta"][nm]
        is_emb = nm.endswith("embed_tokens")
        planes = R["idx"][nm]
        if any(p is None for p in planes):
            raise K.Vq2Error(f"{nm}: missing index plane")
        mods[nm] = PackedLinear(m["shape"], m["cfg"], m["tag"], planes, _as_tensor(R["scales"][nm]),
                                cb_emb if is_emb else cb_lin, device)
        if is_emb:
            emb = mods[nm]
    if emb is not None and tie_embeddings:
        mods["lm_head"] = PackedLMHead(emb)
    return mods
