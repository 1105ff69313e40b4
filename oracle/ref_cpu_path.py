"""The reference's CPU path for the decode projections, restated in torch --
TEST INFRASTRUCTURE / CPU BASELINE ONLY (bench.py's cpu_baseline leg).

Restates, in fp32 on the host:
* ``PackedLinear.forward``'s non-fused fallback (vq2/runtime.py:105-110):
  ``xr = rot.fwd(x)`` (vq2/vq.py:74-76: x[perm] * sign, blockwise ``@ H``,
  ``* hb**-0.5``), then ``weight_rows`` (vq2/runtime.py:82-89: F.embedding of
  the decoded codes into the codebooks, summed over stages, times the row
  scale), then ``F.linear``;
* the CPU twins of the grouped kernels ``vq_moe_parallel_gate_up_cpu`` /
  ``vq_moe_parallel_down_cpu`` (vq2/paged_runtime.py:19-41): per expert,
  ``cb[idx & 0xFFFF]`` gather, ``einsum('org,rg->o')``, ``* scale * rs``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def hadamard(n: int) -> torch.Tensor:
    H = torch.ones(1, 1)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H


class CpuRot:
    def __init__(self, perm, sign, hb):
        self.perm = perm.long() if perm is not None else None
        self.sign = sign.float() if sign is not None else None
        self.hb = hb
        self.H = hadamard(hb)

    def fwd(self, x):
        v = x.float()
        if self.perm is not None:
            v = v[..., self.perm]
        if self.sign is not None:
            v = v * self.sign
        sh = v.shape
        y = v.reshape(*sh[:-1], sh[-1] // self.hb, self.hb) @ self.H
        return (y * self.hb ** -0.5).reshape(sh)


def packed_linear_fallback(x, rot: CpuRot, idx0, idx1, cb0, cb1, scale):
    """fp32 y = F.linear(rot.fwd(x), W) with W rebuilt from the index planes."""
    xr = rot.fwd(x)
    ix = idx0.to(torch.int32) & 0xFFFF
    W = F.embedding(ix.long(), cb0.float())
    if idx1 is not None:
        i1 = idx1.to(torch.int32)
        if idx1.dtype != torch.uint8:
            i1 = i1 & 0xFFFF
        W = W + F.embedding(i1.long(), cb1.float())
    W = W.reshape(idx0.shape[0], -1) * scale.float()[:, None]
    return F.linear(xr, W)


def moe_gate_up_cpu(xr, slots, pool_idx, cb, pool_scale, OUT=1024, NG=256, rs=1.0):
    xg = xr.view(NG, 8).float()
    y = torch.empty(slots.shape[0], OUT)
    for k in range(slots.shape[0]):
        s = int(slots[k])
        idx = (pool_idx[s].to(torch.int32) & 0xFFFF).long()
        rec = cb[idx]
        acc = torch.einsum("org,rg->o", rec, xg)
        y[k] = acc.float() * pool_scale[s].float() * rs
    return y


def moe_down_cpu(act_r, slots, pool_idx, cb, pool_scale, OUT=2048, NG=64, rs=1.0):
    y = torch.empty(slots.shape[0], OUT)
    for k in range(slots.shape[0]):
        s = int(slots[k])
        idx = (pool_idx[s].to(torch.int32) & 0xFFFF).long()
        rec = cb[idx]
        acc = torch.einsum("org,rg->o", rec, act_r[k].view(NG, 8).float())
        y[k] = acc.float() * pool_scale[s].float() * rs
    return y
