"""The one-launch sorted MoE's bounded waits (gate_up and down in one launch,
hidden 2048 / intermediate 512), their give-up path forced from the host:
vq2_sorted_moe_set_wait shortens the bound and raises the gate_up count the
down workgroups wait for beyond what the gate_up part can reach.  Every
kernel still exits normally (the waits are bounded), the pairs that gave up
are NaN, and the status word in the workspace header says which wait gave
up (kernels.vq_sorted_moe_status).  Nothing here can hang: each wait ends
after at most 64 polls of ~1 us.  Afterwards the production bound is back
and the same call matches the oracle with the status word clear."""
import pytest
import torch

from compressai_amd import kernels as K, synth
from oracle import vq2_oracle as O

pytestmark = pytest.mark.gpu


def _layer(dev, E=16, k=4):
    from compressai_amd.moe import MoELayer

    cb = synth.codebook(9950)
    gu = synth.indices16(9952, (E + 1, 1024, 256))
    gus = synth.scales(9953, (E + 1, 1024))
    dn = synth.indices16(9962, (E + 1, 2048, 64))
    dns = synth.scales(9963, (E + 1, 2048))
    gate = synth.activations(9951, 2048) * 0.02
    layer = MoELayer(gu.to(dev), gus.to(dev), dn.to(dev), dns.to(dev), cb.to(dev), gate.to(dev), top_k=k)
    return layer, cb, gu, gus, dn, dns


def test_one_launch_wait_give_up_is_observable(dev):
    layer, cb, gu, gus, dn, dns = _layer(dev)
    m = layer.experts_mod
    assert m.sorted_gu is not None
    T, P = 2, 5
    h = synth.activations(9954, (T, 2048), dtype=torch.float16).to(dev)
    ids = torch.tensor([[3, 0, 11, 7, 16], [5, 3, 2, 9, 16]], dtype=torch.int32, device=dev)
    w = torch.softmax(synth.activations(9955, (T, P)).float(), -1).to(dev)
    logits = synth.activations(9956, (T, 16), dtype=torch.float16).to(dev)
    rh, ri = m._rots()
    torch.cuda.synchronize()
    assert K.vq_sorted_moe_status(dev, clear=True) in (0, 1, 2, 3)
    try:
        # ids given: only the count wait; its target is one more than the
        # pair's gate_up workgroups
        K.vq_sorted_moe_set_wait(max_polls=64, extra_arrivals=1)
        print("case: count wait, 64 polls, unreachable target", flush=True)
        out = m.experts(h, ids, w)
        torch.cuda.synchronize()
        assert torch.isnan(out).all()
        assert K.vq_sorted_moe_status(dev) == K.MOE_WAIT_COUNT
        assert m.wait_errors(clear=True) == K.MOE_WAIT_COUNT and m.wait_errors() == 0
        # router built in, no polls at all: the id wait and the count wait
        # both give up at once
        K.vq_sorted_moe_set_wait(max_polls=0, extra_arrivals=0)
        print("case: router, 0 polls", flush=True)
        out2, rid, rw = K.vq_sorted_moe(h, m.sorted_gu, m.gate_up_scale, m.sorted_dn, m.down_scale, m.cb16, rh, ri,
                                        logits=logits, top_k=4, shared_id=16, shared_gate=layer.shared_gate)
        torch.cuda.synchronize()
        assert torch.isnan(out2).all()
        assert layer.wait_errors(clear=True) == K.MOE_WAIT_ID | K.MOE_WAIT_COUNT
        # the router's own outputs are unaffected by the waits
        sid, sw = layer.route(h, logits)
        assert torch.equal(rid.cpu(), sid.cpu().to(torch.int32)) and torch.equal(rw.cpu(), sw.cpu())
    finally:
        K.vq_sorted_moe_set_wait()
    # production bound: the same calls are right and leave the word clear
    print("case: production bound", flush=True)
    out = m.experts(h, ids, w)
    out2 = layer(h, logits)
    torch.cuda.synchronize()
    assert K.vq_sorted_moe_status(dev) == 0
    ph, sh = m.rot_h.perm.cpu().numpy(), m.rot_h.sign.float().cpu().numpy()
    pi, si = m.rot_i.perm.cpu().numpy(), m.rot_i.sign.float().cpu().numpy()
    ref = O.moe_experts(h.cpu(), ids.cpu().numpy(), w.cpu().numpy(),
                        lambda e: (gu[e], None, gus[e], dn[e], None, dns[e]), cb, None, ph, sh, pi, si)
    assert O.max_rel_err(out.cpu().numpy(), ref) < 1e-3
    assert torch.isfinite(out2).all()
