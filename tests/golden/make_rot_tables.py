"""Writes tests/golden/rot_tables.npz: the permutation and sign tables of the
incoherence rotation for the tags the MoE runtime uses (and one 6144-point
dense-path tag), drawn as the reference's Rot draws them (vq2/vq.py:40-54):
seed = int(md5(tag)[:8], 16); g = torch.Generator().manual_seed(seed);
perm = torch.randperm(n, generator=g); sign = 2 * torch.randint(0, 2, (n,),
generator=g) - 1.  The draws depend on torch's CPU generator, so the fixture
pins them across machines and torch builds (tests/test_host.py and the GPU
test that builds the tables on the device both compare against it).

Run from the repository root:  python tests/golden/make_rot_tables.py
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import torch

TAGS = [("moe_expert_2048", 2048), ("moe_expert_512", 512), ("layers.0.mlp.down_proj", 6144)]


def draw(tag: str, n: int):
    seed = int(hashlib.md5(tag.encode()).hexdigest()[:8], 16)
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(n, generator=g)
    sign = torch.randint(0, 2, (n,), generator=g) * 2 - 1
    return seed, perm.numpy().astype(np.int16), sign.numpy().astype(np.int8)


def main():
    out = {}
    for tag, n in TAGS:
        seed, perm, sign = draw(tag, n)
        out[f"{tag}|{n}|seed"] = np.array([seed], np.int64)
        out[f"{tag}|{n}|perm"] = perm
        out[f"{tag}|{n}|sign"] = sign
    path = Path(__file__).resolve().parent / "rot_tables.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes), torch {torch.__version__}")


if __name__ == "__main__":
    main()
