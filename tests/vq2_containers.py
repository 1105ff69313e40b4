"""Test helpers: fixed-width packing and reference-shaped .vq2 containers
(the dict layout of vq2/export.py:88-118), built independently of the
product code."""
import numpy as np
import torch


def pack_fixed(sym, bits):
    """Little-endian fixed-width packing, built bit by bit (independent of
    the byte formulas of the oracle and the kernel); 4- and 12-bit streams
    are padded to whole symbol pairs as vq2/export.py:39-53 does."""
    sym = np.asarray(sym, dtype=np.int64)
    if bits in (4, 12) and len(sym) % 2:
        sym = np.append(sym, 0)
    nbits = len(sym) * bits
    out = np.zeros((nbits + 7) // 8, np.uint8)
    bitpos = np.arange(len(sym))[:, None] * bits + np.arange(bits)[None, :]
    vals = (sym[:, None] >> np.arange(bits)[None, :]) & 1
    np.add.at(out, bitpos.reshape(-1) // 8, (vals.reshape(-1) << (bitpos.reshape(-1) % 8)).astype(np.uint8))
    return out[: (nbits + 7) // 8]


def key(cfg, i):
    return "_".join(str(b) for b in cfg[: i + 1])


def make_container(mats, codebooks, codebooks_embed=None, seed=0):
    """mats: {name: (shape, cfg, tag)} -> (container dict, planes) with random
    codes: planes[name] = [stage-0 codes (uint16 values, int64), ...];
    streams fixed-width packed in names order, numpy scales and counts as
    the reference writes them."""
    rng = np.random.default_rng(seed)
    names = list(mats)
    planes, streams = {}, {}
    for nm in names:
        (out, n), cfg, _ = mats[nm]
        planes[nm] = [rng.integers(0, 1 << b, (out, n // 8), dtype=np.int64) for b in cfg]
        for i, b in enumerate(cfg):
            streams.setdefault(key(cfg, i), []).append(planes[nm][i].reshape(-1))
    C = {"names": names,
         "meta": {nm: dict(shape=mats[nm][0], cfg=mats[nm][1], tag=mats[nm][2]) for nm in names},
         "streams": {},
         "scales": {nm: (rng.random(mats[nm][0][0]) + 0.5).astype(np.float16) for nm in names}}
    for k, lst in streams.items():
        bits = int(k.split("_")[-1])
        allsym = np.concatenate(lst)
        C["streams"][k] = dict(sizes=[len(a) for a in lst], counts=np.bincount(allsym, minlength=1 << bits)
                               .astype(np.uint32), bits=bits, mode="fixed",
                               fixed=torch.from_numpy(pack_fixed(allsym, bits)))
    C["codebooks"] = {k: v.half() for k, v in codebooks.items()}
    C["codebooks_embed"] = {k: v.half() for k, v in (codebooks_embed or {}).items()}
    C["dense"] = {"model.norm.weight": torch.ones(8, dtype=torch.bfloat16)}
    return C, planes
