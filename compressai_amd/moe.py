"""MoE expert layer of the decode path on a device-resident expert pool.

``ResidentMoEExperts`` is the drop-in for the reference's resident expert
module ``PackedMoEExpertUniversal`` (vq2/load_and_test_full_35b.py:26-95):
``forward(hidden_states [T, H], topk_idx [T, K], topk_weights [T, K])``
returns ``[T, H]``, computing per token t and expert e = topk_idx[t, k]

    xr  = rot_H.fwd(h_t)                                   (RHT, hb = 2048)
    gu  = VQ(gate_up[e]) xr                                 ([2I], gate | up)
    act = rot_I.fwd(silu(gu[:I]) * gu[I:])                  (RHT, hb = I)
    out_t = sum_k w[t, k] * VQ(down[e]) act

(vq2/paged_runtime.py:495-510).  Instead of the reference's per-token Python
loop (load_and_test_full_35b.py:75-95) every token and expert goes into two
launches: grouped gate_up with the H-point RHT built in each workgroup's LDS,
then SwiGLU + I-point RHT (again in LDS) + grouped down + weighted combine.
Expert ids are read on the device: no ``.tolist()`` and no host
synchronisation.

``MoELayer`` adds the router (softmax -> top-k -> renormalise on given
logits) and the shared expert with its sigmoid gate (transformers 5.15.0
``Qwen3_5MoeTopKRouter`` / ``Qwen3_5MoeSparseMoeBlock``), the shared expert
living in the same pool at id ``n_routed``.  The whole layer is two
launches and no host synchronisation.

Intermediates are fp32 by default (the parity contract); ``act_dtype`` may
select bf16 to follow the reference's cast points instead.

On the GPU, with fp16 / bf16 codebooks and fp32 intermediates, both modules
also keep a code-sorted copy of the expert pools (``kernels.SortedPool``,
packed once at construction, ~3.06 bytes per code against the pools' 2) and
run the experts over it, so a wave's centroid gathers share codebook lines:
at hidden 2048 / intermediate 512 (the 35B-A3B shape) gate_up (router built
in for ``MoELayer``) and down (SwiGLU + RHT in its prologue) are one launch,
followed by the combine launch; other widths take a separate down launch.
The reference pools stay the public format and serve ``act_dtype`` bf16,
more than 256 routed experts and the paged feed; a caller that needs none
of these frees them with ``release_reference_pools()`` (resident index
memory then ~3.06 instead of ~5.06 bytes per code; ``sorted_layout=False``
keeps only the 2-byte pools, on the gather kernels).  The down pool is
sorted twice where taller chunks fit its 16-bit positions (the 35B shape:
5 chunks of 410 rows besides 9 of 228), the taller copy for T >= 2
(``release_tall_down()`` drops it, ~1.2 bytes per down code).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import kernels as K
from .rot import get_rot


def _tall_rows(rows, ng, default_rows):
    """Chunk height of the taller down pool: the fewest chunks of at most 511
    rows that 16-bit positions hold (the down pool of the 35B shape, 2048
    rows of 64 groups: 5 chunks of 410 rows); None unless that is at least
    a quarter taller than default_rows (the pool's memory buys little
    otherwise)."""
    gb = max(0, (int(ng) - 1).bit_length())
    if gb > 15:
        return None
    rmax = min((1 << (16 - gb)) - 1, 511)
    n = -(-int(rows) // rmax)
    r = -(-int(rows) // n)
    return r if 4 * r >= 5 * int(default_rows) else None


class ResidentMoEExperts(nn.Module):
    """Resident expert pool of one MoE layer.

    ``ResidentMoEExperts(q_gate_up, q_down, cb16, device)`` is the
    reference's constructor (``PackedMoEExpertUniversal``,
    vq2/load_and_test_full_35b.py:31-47): the quantized dicts' stage-1 index
    planes are viewed as the pools ``[E, 2I, H/8]`` / ``[E, H, I/8]`` and their
    row scales rounded to bf16, exactly as the reference does.  ``from_pools``
    takes ready device pools (any scale dtype, kept as given)."""

    def __init__(self, q_gate_up, q_down, cb16, device="cuda", *, num_experts=256, hidden_dim=2048,
                 intermediate_dim=512, rot_h=None, rot_i=None, act_dtype=torch.float32, out_dtype=None,
                 sorted_layout=None):
        super().__init__()
        E, H, I = int(num_experts), int(hidden_dim), int(intermediate_dim)
        gu_idx = q_gate_up["idx"][0]
        dn_idx = q_down["idx"][0]
        if gu_idx.numel() != E * 2 * I * (H // 8) or dn_idx.numel() != E * H * (I // 8):
            raise K.Vq2Error(f"quantized expert planes of {gu_idx.numel()} / {dn_idx.numel()} codes do not hold "
                             f"{E} experts of gate_up [{2 * I}, {H}] / down [{H}, {I}]")
        self._setup(gu_idx.view(E, 2 * I, H // 8).to(device),
                    q_gate_up["scale"].view(E, 2 * I).to(device=device, dtype=torch.bfloat16),
                    dn_idx.view(E, H, I // 8).to(device),
                    q_down["scale"].view(E, H).to(device=device, dtype=torch.bfloat16),
                    cb16, rot_h, rot_i, act_dtype, out_dtype, sorted_layout)

    @classmethod
    def from_pools(cls, gate_up_idx, gate_up_scale, down_idx, down_scale, cb16, rot_h=None, rot_i=None,
                   act_dtype=torch.float32, out_dtype=None, sorted_layout=None):
        """Pools already on the device: gate_up_idx [E, 2I, H/8], down_idx
        [E, H, I/8] (int16), scales [E, 2I] / [E, H] in any float dtype."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self._setup(gate_up_idx, gate_up_scale, down_idx, down_scale, cb16, rot_h, rot_i, act_dtype, out_dtype,
                    sorted_layout)
        return self

    def _setup(self, gate_up_idx, gate_up_scale, down_idx, down_scale, cb16, rot_h, rot_i, act_dtype, out_dtype,
               sorted_layout=None):
        E, gu_rows, ng_h = gate_up_idx.shape
        E2, hidden, ng_i = down_idx.shape
        if E2 != E or gu_rows != 2 * ng_i * 8 or hidden != ng_h * 8:
            raise K.Vq2Error("inconsistent gate_up/down pool shapes")
        self.num_experts = E
        self.hidden_dim = hidden
        self.intermediate_dim = ng_i * 8
        dev = gate_up_idx.device
        self.gate_up_idx = gate_up_idx
        self.gate_up_scale = gate_up_scale
        self.down_idx = down_idx
        self.down_scale = down_scale
        self.cb16 = cb16
        self.rot_h = rot_h if rot_h is not None else get_rot("moe_expert_2048", hidden, dev)
        self.rot_i = rot_i if rot_i is not None else get_rot("moe_expert_512", self.intermediate_dim, dev)
        self.act_dtype = act_dtype
        self.out_dtype = out_dtype
        # code-sorted copies of the pools (the experts' batch-1 and small-T path)
        use = sorted_layout if sorted_layout is not None else (
            dev.type == "cuda" and act_dtype == torch.float32 and cb16.dtype in (torch.float16, torch.bfloat16)
            and hidden % 64 == 0 and self.intermediate_dim % 64 == 0 and hidden <= 8192)
        self.sorted_gu = K.SortedPool(gate_up_idx, device=dev) if use else None
        self.sorted_dn = K.SortedPool(down_idx, device=dev) if use else None
        # the down pool again in taller chunks, for T >= 2 (_down_pool)
        tall = _tall_rows(hidden, ng_i, self.sorted_dn.rows_per_chunk) if use else None
        self.sorted_dn_tall = K.SortedPool(down_idx, device=dev, rows_per_chunk=tall) if tall else None

    def _down_pool(self, T):
        """The down pool for T tokens: from T = 2 on the taller chunks, whose
        fewer, longer workgroups gather fewer codebook lines per instruction
        (20 layers of the 35B shape, down in 5 chunks of 410 rows against 9
        of 228: T = 2 / 3 / 4 / 8 28.8 / 33.5 / 40.7 / 59.2 us per layer
        against 29.2 / 35.5 / 41.6 / 64.3; T = 1 20.6 against 19.8, so T = 1
        keeps the default chunks)."""
        if T >= 2 and self.sorted_dn_tall is not None:
            return self.sorted_dn_tall
        return self.sorted_dn

    def release_tall_down(self):
        """Drop the taller down pool (~1.2 bytes per down code less resident);
        every T then runs on the default chunks."""
        self.sorted_dn_tall = None

    def release_reference_pools(self):
        """Drop the reference index pools once the sorted copies exist (the
        row scales stay: both layouts read them).  Afterwards only the
        sorted path runs; act_dtype bf16 and n_routed > 256 raise."""
        if self.sorted_gu is None:
            raise K.Vq2Error("release_reference_pools: no sorted copy to run on")
        self.gate_up_idx = None
        self.down_idx = None

    def _reference_pools(self):
        if self.gate_up_idx is None:
            raise K.Vq2Error("the reference pools were released (release_reference_pools); only the sorted "
                             "path runs")

    def wait_errors(self, clear=False) -> int:
        """Wait-timeout bits of the one-launch sorted MoE on the current
        stream (kernels.vq_sorted_moe_status; a host synchronisation)."""
        return K.vq_sorted_moe_status(self.cb16.device, clear=clear)

    def _rots(self):
        rh, ri = self.rot_h, self.rot_i
        return (rh._perm32, rh._sign8, rh.hb, rh.scale), (ri._perm32, ri._sign8, ri.hb, ri.scale)

    def nbytes(self):
        """Resident bytes: index pools, scales and the sorted copies."""
        own = sum(t.numel() * t.element_size() for t in (self.gate_up_idx, self.gate_up_scale, self.down_idx,
                                                          self.down_scale) if t is not None)
        return own + sum(p.nbytes() for p in (self.sorted_gu, self.sorted_dn, self.sorted_dn_tall) if p is not None)

    def experts(self, h, ids, w, out=None):
        """h [T, H] (unrotated hidden states), ids [T, P] int32/int64,
        w fp32 [T, P] -> [T, H].  Sorted pools: gate_up and down (SwiGLU +
        RHT in its prologue) in one launch at the 35B shape, then the combine;
        otherwise two launches, gate_up with the H-point RHT fused, then
        SwiGLU + I-point RHT + down + weighted combine."""
        if self.sorted_gu is not None:
            rh, ri = self._rots()
            return K.vq_sorted_moe(h, self.sorted_gu, self.gate_up_scale, self._down_pool(h.shape[0]), self.down_scale,
                                   self.cb16, rh, ri, ids=ids, w=w, out=out, out_dtype=self.out_dtype or torch.float32)
        self._reference_pools()
        T, P = ids.shape
        I = self.intermediate_dim
        y_gu = torch.empty((T * P, 2 * I), dtype=self.act_dtype, device=h.device)
        K.vq_moe_gate_up_rht(h, ids, self.gate_up_idx, self.cb16, self.gate_up_scale, y_gu, OUT=2 * I,
                             NG=self.hidden_dim // 8, perm=self.rot_h._perm32, sign=self.rot_h._sign8,
                             hb=self.rot_h.hb, rht_scale=self.rot_h.scale)
        return K.vq_moe_down_swiglu_combine(y_gu, ids, w, self.down_idx, self.cb16, self.down_scale,
                                            OUT=self.hidden_dim, NG=I // 8, perm=self.rot_i._perm32,
                                            sign=self.rot_i._sign8, hb=self.rot_i.hb, rht_scale=self.rot_i.scale,
                                            out=out, out_dtype=self.out_dtype or torch.float32)

    def forward(self, hidden_states, topk_idx, topk_weights):
        h = hidden_states.reshape(-1, self.hidden_dim).contiguous()
        ids = topk_idx.reshape(h.shape[0], -1)
        if ids.dtype not in (torch.int32, torch.int64):
            ids = ids.to(torch.int32)
        w = topk_weights.reshape(ids.shape).to(torch.float32).contiguous()
        out = self.experts(h, ids.contiguous(), w)
        return out.to(self.out_dtype or hidden_states.dtype)


class MoELayer(nn.Module):
    """Router + top-k routed experts + gated shared expert, one pool.

    pools: gate_up_idx [E+1, 2I, H/8], down_idx [E+1, H, I/8] (int16), scales
    [E+1, 2I] / [E+1, H]; id E is the shared expert.  shared_gate [H]."""

    def __init__(self, gate_up_idx, gate_up_scale, down_idx, down_scale, cb16, shared_gate, top_k=8,
                 n_routed=None, rot_h=None, rot_i=None, act_dtype=torch.float32, out_dtype=torch.float32,
                 sorted_layout=None):
        super().__init__()
        self.experts_mod = ResidentMoEExperts.from_pools(gate_up_idx, gate_up_scale, down_idx, down_scale, cb16,
                                                         rot_h, rot_i, act_dtype, out_dtype, sorted_layout)
        self.n_routed = gate_up_idx.shape[0] - 1 if n_routed is None else int(n_routed)
        self.top_k = int(top_k)
        self.shared_gate = shared_gate
        self.out_dtype = out_dtype
        # down projection: one launch (SwiGLU + RHT in every workgroup) or a
        # separate SwiGLU + RHT launch followed by the grouped down + combine
        self.fused_down = True

    def route(self, h, router_logits):
        return K.vq_router_topk(router_logits, self.top_k, h, self.shared_gate, shared_id=self.n_routed)

    def wait_errors(self, clear=False) -> int:
        return self.experts_mod.wait_errors(clear)

    def forward(self, h, router_logits):
        """Sorted pools: router + gate_up and down (SwiGLU + RHT prologue) in
        one launch at the 35B shape, then the combine.  Otherwise two
        launches: router + gate_up (+ RHT), then SwiGLU + RHT + down +
        combine."""
        m = self.experts_mod
        h2 = h.reshape(-1, m.hidden_dim).contiguous()
        T = h2.shape[0]
        if m.sorted_gu is not None and self.n_routed <= 256:
            rh, ri = m._rots()
            out, _, _ = K.vq_sorted_moe(h2, m.sorted_gu, m.gate_up_scale, m._down_pool(T), m.down_scale, m.cb16, rh, ri,
                                        logits=router_logits.reshape(T, -1), top_k=self.top_k,
                                        shared_id=self.n_routed, shared_gate=self.shared_gate,
                                        out_dtype=m.out_dtype or torch.float32)
            return out
        m._reference_pools()
        I = m.intermediate_dim
        P = self.top_k + 1
        y_gu = torch.empty((T * P, 2 * I), dtype=m.act_dtype, device=h2.device)
        ids, w = K.vq_moe_router_gate_up_rht(h2, router_logits.reshape(T, -1), self.top_k, m.gate_up_idx, m.cb16,
                                             m.gate_up_scale, y_gu, OUT=2 * I, NG=m.hidden_dim // 8,
                                             shared_gate=self.shared_gate, shared_id=self.n_routed,
                                             perm=m.rot_h._perm32, sign=m.rot_h._sign8, hb=m.rot_h.hb,
                                             rht_scale=m.rot_h.scale)
        if self.fused_down:
            return K.vq_moe_down_swiglu_combine(y_gu, ids, w, m.down_idx, m.cb16, m.down_scale, OUT=m.hidden_dim,
                                                NG=I // 8, perm=m.rot_i._perm32, sign=m.rot_i._sign8,
                                                hb=m.rot_i.hb, rht_scale=m.rot_i.scale,
                                                out_dtype=m.out_dtype or torch.float32)
        act = K.vq_swiglu_rht(y_gu, I, m.rot_i._perm32, m.rot_i._sign8, m.rot_i.hb, m.rot_i.scale)
        return K.vq_moe_down_combine(act, ids, w, m.down_idx, m.cb16, m.down_scale, OUT=m.hidden_dim, NG=I // 8,
                                     out_dtype=m.out_dtype or torch.float32)


# the reference's name for the resident expert module
# (vq2/load_and_test_full_35b.py:26, vq2/inferencia_35b.py:22)
PackedMoEExpertUniversal = ResidentMoEExperts
