"""The reference's CPU path for the decode projections and the MoE layer,
restated in torch -- TEST INFRASTRUCTURE / CPU BASELINE ONLY (the
``cpu_baseline`` legs of bench.py, and tests/test_host.py, which pins these
functions against the C oracle).

Restates, on the host (paths relative to the reference repository):
* ``PackedLinear.forward``'s non-fused fallback (vq2/runtime.py:105-110):
  ``xr = rot.fwd(x)`` (vq2/vq.py:74-76: x[perm] * sign, blockwise ``@ H``,
  ``* hb**-0.5``), then ``weight_rows`` (vq2/runtime.py:82-89: F.embedding of
  the decoded codes into the codebooks, summed over stages, times the row
  scale), then ``F.linear`` -- in fp32;
* the CPU twins of the grouped kernels ``vq_moe_parallel_gate_up_cpu`` /
  ``vq_moe_parallel_down_cpu`` (vq2/paged_runtime.py:19-41): per slot,
  ``cb[idx & 0xFFFF]`` gather ([OUT, NG, 8]), ``einsum('org,rg->o')`` with the
  activation in the codebook dtype, then ``acc.float() * scale * rs``; fed
  fp32 codebooks as scratch/test_cpu_paged_moe.py:37-53 does;
* the MoE layer composed from them, token by token (the reference's T > 1
  loop, vq2/load_and_test_full_35b.py:75-95, whose body is the T == 1 path of
  vq2/paged_runtime.py:491-511, with RS_2048 = RS_512 = 1 because Rot already
  scales), plus the router and the gated shared expert of transformers 5.15.0
  (``Qwen3_5MoeTopKRouter``: softmax in fp32, top-k, renormalise;
  ``Qwen3_5MoeSparseMoeBlock``: + sigmoid(shared_gate . h) * shared_expert(h)).
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
    """Rot.fwd in fp32 (vq2/vq.py:66-76): x[..., perm] * sign, blocks @ H, * hb**-0.5."""

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
    """vq_moe_parallel_gate_up_cpu: y[k] = (einsum(cb[pool[s_k]], xr) * scale[s_k] * rs), fp32 [K, OUT]."""
    xg = xr.reshape(NG, 8).to(cb.dtype)
    y = torch.empty(len(slots), OUT, dtype=torch.float32)
    for k, s in enumerate(slots):
        s = int(s)
        idx = (pool_idx[s].to(torch.int32) & 0xFFFF).long()
        acc = torch.einsum("org,rg->o", cb[idx], xg)
        y[k] = acc.float() * pool_scale[s].float() * rs
    return y


def moe_down_cpu(act_r, slots, pool_idx, cb, pool_scale, OUT=2048, NG=64, rs=1.0):
    """vq_moe_parallel_down_cpu: as moe_gate_up_cpu with one activation per slot."""
    y = torch.empty(len(slots), OUT, dtype=torch.float32)
    for k, s in enumerate(slots):
        s = int(s)
        idx = (pool_idx[s].to(torch.int32) & 0xFFFF).long()
        acc = torch.einsum("org,rg->o", cb[idx], act_r[k].reshape(NG, 8).to(cb.dtype))
        y[k] = acc.float() * pool_scale[s].float() * rs
    return y


def router_topk_cpu(logits, k):
    """Qwen3_5MoeTopKRouter on given logits: (ids [T, k] int64, w [T, k] fp32)."""
    p = torch.softmax(logits.float(), dim=-1)
    w, ids = torch.topk(p, k, dim=-1)
    return ids, w / w.sum(-1, keepdim=True)


def moe_layer_cpu(h, logits, cb, gu_pool, gu_scale, dn_pool, dn_scale, shared_gate, rot_h: CpuRot, rot_i: CpuRot,
                  top_k=8, shared_id=None):
    """One MoE layer on the host, token by token: router -> rot_h.fwd(h_t) ->
    grouped gate_up over the routed slots (+ the shared expert, pool id
    ``shared_id``) -> silu(gate) * up -> rot_i.fwd -> grouped down -> the
    weighted sum + sigmoid(shared_gate . h_t) * shared output.  fp32 [T, H]."""
    T, H = h.shape
    I = dn_pool.shape[-1] * 8
    ids, w = router_topk_cpu(logits, top_k)
    out = torch.empty(T, H, dtype=torch.float32)
    for t in range(T):
        slots = ids[t].tolist() + ([shared_id] if shared_id is not None else [])
        xr = rot_h.fwd(h[t])
        y_gu = moe_gate_up_cpu(xr, slots, gu_pool, cb, gu_scale, OUT=2 * I, NG=H // 8)
        act = F.silu(y_gu[:, :I]) * y_gu[:, I:]
        y_dn = moe_down_cpu(rot_i.fwd(act), slots, dn_pool, cb, dn_scale, OUT=H, NG=I // 8)
        o = (y_dn[:top_k] * w[t][:, None]).sum(0)
        if shared_id is not None:
            o = o + torch.sigmoid(shared_gate.float() @ h[t].float()) * y_dn[top_k]
        out[t] = o
    return out
