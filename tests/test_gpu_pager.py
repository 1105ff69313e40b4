"""GPU tests of the device-resident expert pager (vq2_pager_step /
vq2_pager_copy through the C ABI): after every step the device tables equal
a Python model of the same paging rule (resident experts keep their slots;
the distinct missing experts, in pair order, take the slots the step does
not use, least recently used first, ties to the lower slot), the pool slots
hold the container records bit for bit (scales rounded fp16 -> bf16 as
torch rounds them), errors are flagged instead of read out of bounds, and
PagedMoEExperts on device tables gives the resident pool's outputs, eagerly
and replayed from a captured HIP graph."""
import numpy as np
import pytest
import torch

from compressai_amd import paged, synth

pytestmark = pytest.mark.gpu


def _container(tmp_path, E, gu=(32, 16), dn=(64, 8), seed=0):
    g = torch.Generator().manual_seed(seed)
    gui = torch.randint(-32768, 32768, (E, *gu), generator=g, dtype=torch.int32).to(torch.int16)
    gus = (torch.rand(E, gu[0], generator=g) * 3 - 1.5).to(torch.float16)
    dni = torch.randint(-32768, 32768, (E, *dn), generator=g, dtype=torch.int32).to(torch.int16)
    dns = (torch.rand(E, dn[0], generator=g) * 3 - 1.5).to(torch.float16)
    path = tmp_path / "m.vq2m"
    paged.write_vq2m(path, [gui], [gus], [dni], [dns])
    return paged.Vq2mStore(path), (gui, gus, dni, dns)


class LruModel:
    """The paging rule of vq2_pager_step, step by step on the host."""

    def __init__(self, E, C):
        self.E, self.C = E, C
        self.slot_of = [-1] * E
        self.expert_of = [-1] * C
        self.stamp = [-1] * C
        self.clock = 0
        self.hits = self.misses = 0
        self.errors = 0

    def step(self, ids):
        self.clock += 1
        pe = [e if 0 <= e < self.E else -1 for e in ids]
        if any(e < 0 for e in pe):
            self.errors |= 1
        for e in pe:
            if e >= 0 and self.slot_of[e] >= 0:
                self.stamp[self.slot_of[e]] = self.clock
        miss = []
        for e in pe:
            if e >= 0 and self.slot_of[e] < 0 and e not in miss:
                miss.append(e)
        elig = sorted((s for s in range(self.C) if self.stamp[s] != self.clock), key=lambda s: (self.stamp[s], s))
        served = min(len(miss), len(elig))
        if served < len(miss):
            self.errors |= 2
        for r in range(served):
            old = self.expert_of[elig[r]]
            if old >= 0:
                self.slot_of[old] = -1
        for r in range(served):
            e, v = miss[r], elig[r]
            self.slot_of[e], self.expert_of[v], self.stamp[v] = v, e, self.clock
        self.hits += sum(e >= 0 for e in pe) - len(miss)
        self.misses += len(miss)
        return [self.slot_of[e] if e >= 0 else -1 for e in pe], [(miss[r], elig[r]) for r in range(served)]


@pytest.mark.parametrize("C,T", [(12, 2), (7, 1)])   # 7 slots: the stamps padded to 8 in LDS
@pytest.mark.parametrize("sorted_layout", [False, True])
def test_device_pager_tables_follow_the_model(dev, tmp_path, sorted_layout, C, T):
    E, P = 40, 5
    store, (gui, gus, dni, dns) = _container(tmp_path, E)
    pager = paged.ExpertPager(store, 0, C, dev, device_tables=True, sorted_layout=sorted_layout)
    model = LruModel(E, C)
    g = torch.Generator().manual_seed(5)
    for step in range(60):
        hot = torch.randint(0, 10, (T * P,), generator=g)          # a few hot experts ...
        cold = torch.randint(0, E, (T * P,), generator=g)          # ... and the rest
        ids = torch.where(torch.rand(T * P, generator=g) < 0.6, hot, cold).view(T, P)
        ids = ids.to(torch.int32 if step % 2 else torch.int64)
        slots = pager.step(ids.to(dev)).cpu().view(-1).tolist()
        want, copies = model.step(ids.view(-1).tolist())
        assert slots == want, step
        assert pager.d_slot_of.cpu().tolist() == model.slot_of, step
        assert pager.d_expert_of.cpu().tolist() == model.expert_of, step
        assert pager.d_stamp.cpu().tolist() == model.stamp, step
        st = pager.d_state.cpu().tolist()
        assert st[0] == model.clock and st[1] == len(copies) and st[2:] == [model.hits, model.misses, 0], step
    # every resident slot holds its expert's record (sorted: the expert's
    # chunks as the layer's sorted pool packs them)
    if sorted_layout:
        from compressai_amd.kernels import SortedPool

        ref_gu, ref_dn = SortedPool(gui, device="cpu"), SortedPool(dni, device="cpu")
        gw, dw = ref_gu.expert_words(), ref_dn.expert_words()
    for v, e in enumerate(model.expert_of):
        if e < 0:
            continue
        if sorted_layout:
            assert torch.equal(pager.sorted_gu.entries[v * gw:(v + 1) * gw].cpu(), ref_gu.entries[e * gw:(e + 1) * gw])
            assert torch.equal(pager.sorted_dn.entries[v * dw:(v + 1) * dw].cpu(), ref_dn.entries[e * dw:(e + 1) * dw])
        else:
            assert torch.equal(pager.pool_gu_idx[v].cpu(), gui[e])
            assert torch.equal(pager.pool_dn_idx[v].cpu(), dni[e])
        assert torch.equal(pager.pool_gu_scale[v].cpu(), gus[e].to(torch.bfloat16))
        assert torch.equal(pager.pool_dn_scale[v].cpu(), dns[e].to(torch.bfloat16))
    store.close()


def test_device_pager_fp16_scales_and_errors(dev, tmp_path):
    """scale_dtype=None keeps the container's fp16 scales; an id outside the
    layer and a step with more distinct experts than slots give slot -1 and
    set the error bits, leaving the rest of the step served."""
    E, C = 20, 4
    store, (gui, gus, dni, dns) = _container(tmp_path, E, seed=3)
    pager = paged.ExpertPager(store, 0, C, dev, scale_dtype=None, device_tables=True)
    model = LruModel(E, C)
    ids = torch.tensor([[3, E, 7, -1]], dtype=torch.int64)
    slots = pager.step(ids.to(dev)).cpu().view(-1).tolist()
    assert slots == model.step([3, E, 7, -1])[0] and slots[1] == slots[3] == -1
    assert pager.errors == 1
    v = slots[0]
    assert torch.equal(pager.pool_gu_scale[v].cpu(), gus[3]) and pager.pool_gu_scale.dtype == torch.float16
    ids = torch.tensor([[1, 2, 4, 5, 6, 8]], dtype=torch.int32)  # 6 distinct experts, 4 slots
    slots = pager.step(ids.to(dev)).cpu().view(-1).tolist()
    assert slots == model.step(ids.view(-1).tolist())[0]
    assert slots[4] == slots[5] == -1 and all(s >= 0 for s in slots[:4])
    assert pager.errors == 3
    store.close()


@pytest.mark.parametrize("sorted_layout", [False, True])
def test_paged_device_tables_match_resident_pool_and_replay(dev, tmp_path, sorted_layout):
    """PagedMoEExperts(device_tables=True) at the config-4 expert shape,
    6 slots over 16 experts: every step equals the resident pool bit for bit
    (gather kernels on reference-layout slots, or the one-launch sorted MoE
    on a sorted slot pool against the resident sorted pool); a captured graph
    of 4 steps replays them exactly."""
    from compressai_amd.graph import DecodeStepGraph
    from compressai_amd.moe import ResidentMoEExperts

    E = 16
    store, (gui, gus, dni, dns) = _container(tmp_path, E, gu=(1024, 256), dn=(2048, 64), seed=11)
    cb = synth.codebook(4601).to(dev)
    pg = paged.PagedMoEExperts(0, store, cb, capacity=6, device=dev, out_dtype=torch.float32, device_tables=True,
                               sorted_layout=sorted_layout)
    assert pg.pager.sorted_layout == sorted_layout
    bf = torch.bfloat16
    res = ResidentMoEExperts.from_pools(gui.to(dev), gus.to(dev, bf), dni.to(dev), dns.to(dev, bf), cb,
                                        out_dtype=torch.float32, sorted_layout=sorted_layout)
    if sorted_layout:
        # the slot pool has the default chunk heights at every T: so must the reference
        res.release_tall_down()
    g = torch.Generator().manual_seed(4602)
    steps = []
    for step in range(8):
        T = 1 + step % 3
        ids = torch.stack([torch.randperm(E, generator=g)[:2] for _ in range(T)])
        w = torch.softmax(torch.randn(T, 2, generator=g), -1)
        h = synth.activations(4610 + step, (T, 2048), dtype=torch.float16)
        steps.append((h.to(dev), ids.to(dev), w.to(dev)))
        yp = pg(*steps[-1])
        yr = res(*steps[-1])
        assert torch.equal(yp, yr), step
    assert pg.pager.misses > 6 and pg.pager.hits > 0 and pg.pager.errors == 0
    # graph: one step's static buffers, replayed with new ids each time
    h0, i0, w0 = (t.clone() for t in steps[0])
    graph = DecodeStepGraph(lambda h, i, w: pg(h, i, w), [h0, i0, w0])
    for r in range(4):
        ids = torch.stack([torch.randperm(E, generator=g)[:2]]).to(dev)
        h = synth.activations(4700 + r, (1, 2048), dtype=torch.float16).to(dev)
        out = graph(h, ids, w0).clone()
        torch.cuda.synchronize()
        assert torch.equal(out, res(h, ids, w0)), r
    assert pg.pager.errors == 0
    store.close()
