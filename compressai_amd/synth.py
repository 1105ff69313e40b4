"""Seeded synthetic inputs for the VQ2 decode-path workloads.

Every tensor is drawn on the host from ``torch.Generator('cpu')`` so that a
CPU checker and the GPU see identical bits.  Seed convention: workload ``k``
uses ``1000*k + j`` with j = 0 codebook, 1 stage-2 codebook, 2 indices,
3 scales, 4 activations, 5 RHT signs, 6 RHT permutation, 7 router logits,
8 shared-expert gate vector (further draws of one kind add 10*i to j).

Distributions (the workload definitions of the decode path):
  codebooks      fp16 N(0, 1/8)   (variance 1/8), [rows, 8]
  indices        uniform on [0, 65536), stored as int16 bit patterns
  stage-2 uint8  uniform on [0, 256)
  scales         fp16 U(0.5, 1.5)
  activations    fp16 N(0, 1)
  RHT signs      Rademacher, int8 +-1
"""
from __future__ import annotations

import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(int(seed))


def codebook(seed: int, rows: int = 65536, dtype=torch.float16) -> torch.Tensor:
    return (torch.randn(rows, 8, generator=gen(seed)) * (1.0 / 8.0) ** 0.5).to(dtype)


def indices16(seed: int, shape) -> torch.Tensor:
    """uint16 codes stored as int16 bit patterns (code c >= 32768 -> c - 65536)."""
    v = torch.randint(0, 65536, tuple(shape), generator=gen(seed), dtype=torch.int32)
    return torch.where(v >= 32768, v - 65536, v).to(torch.int16)


def indices8(seed: int, shape) -> torch.Tensor:
    return torch.randint(0, 256, tuple(shape), generator=gen(seed), dtype=torch.int32).to(torch.uint8)


def scales(seed: int, rows, dtype=torch.float16) -> torch.Tensor:
    shape = (rows,) if isinstance(rows, int) else tuple(rows)
    return (torch.rand(shape, generator=gen(seed)) + 0.5).to(dtype)


def activations(seed: int, shape, dtype=torch.float16) -> torch.Tensor:
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    return torch.randn(shape, generator=gen(seed)).to(dtype)


def signs(seed: int, n: int) -> torch.Tensor:
    return (torch.randint(0, 2, (n,), generator=gen(seed), dtype=torch.int32) * 2 - 1).to(torch.int8)


def permutation(seed: int, n: int) -> torch.Tensor:
    return torch.randperm(n, generator=gen(seed)).to(torch.int32)


def vq_matrix(seed_base: int, out_rows: int, n: int, bpw: int = 2, draw: int = 0):
    """Index planes and scales of one VQ matrix.  bpw 2 -> (16,), 3 -> (16, 8),
    4 -> (16, 16).  Returns dict(idx0, idx1 or None, scale)."""
    ng = n // 8
    d = 10 * draw
    idx0 = indices16(seed_base + 2 + d, (out_rows, ng))
    idx1 = None
    if bpw == 3:
        idx1 = indices8(seed_base + 2 + d + 100, (out_rows, ng))
    elif bpw == 4:
        idx1 = indices16(seed_base + 2 + d + 100, (out_rows, ng))
    return dict(idx0=idx0, idx1=idx1, scale=scales(seed_base + 3 + d, out_rows))
