"""Paged expert-pool feed for the MoE decode path (reference: vq2/paged_runtime.py).

``Vq2mStore`` reads the ``.vq2m`` container the reference writes
(vq2/pack_35b_to_vq2m.py:22-25, 225-244; reader vq2/paged_runtime.py:49-123):
a 64-byte header ``<4sHHHH QQQQQ 12s`` (magic ``VQ2M``, version 1, layers,
experts, table and meta offsets, payload start), one ``<QIQIQIQI`` entry per
(layer, expert) -- offset and size of the gate_up index plane, its fp16 scales,
the down index plane and its scales -- and a JSON meta block.  Each expert's
four tensors are written back to back, so one read fetches the whole record
(792,576 bytes at the config-4 shape).  ``write_vq2m`` writes the same layout
(for tests and benchmarks).

``PagedMoEExperts`` is the drop-in for ``PagedMoEExpert``
(vq2/paged_runtime.py:316-568): ``forward(hidden_states [T, H], topk_idx
[T, K], topk_weights [T, K])`` over a device pool of ``capacity`` expert
slots managed LRU (``_get_slot``, vq2/paged_runtime.py:415-437).  Where the
reference reads each missing expert synchronously through one reused pinned
buffer and hands the kernels a slot list built element by element, here:

* missing records are read (``os.preadv``) into a ring of pinned staging
  records and copied to their slots on a dedicated copy stream; a staging
  record is reused only after the event of its previous copy has completed;
* the copy stream first waits for the work already queued on the compute
  stream (a slot being evicted may still be read by the previous layer's
  launch), and the compute stream waits for the copies through one event: no
  host synchronisation besides the one read of the routed ids that the
  host-side paging decision needs;
* the slot ids of all (token, expert) pairs go to the device in one copy, and
  the two grouped launches of ``ResidentMoEExperts`` (gate_up with the RHT,
  SwiGLU + RHT + down + combine) run unchanged on the slot pool.  The pool
  holds the row scales in bf16, rounded from the container's fp16 as the
  reference's pools do (vq2/paged_runtime.py:140-173, 340-342);
  ``scale_dtype=None`` keeps the fp16 scales.

Promoted 3 bpw experts (``expert_modes["layer:expert"] == 3``, written by
tools/build_mixed_b2_container.py:50-82, 154-165): their index entries hold
the int16 stage-1 plane followed by the uint8 stage-2 plane of the (16,8)
scheme (1,185,792-byte records at the config-4 shape).  The reference keeps
them resident as dense bf16 weights and runs them through ``F.linear`` per
token (vq2/paged_runtime.py:357-389, 446-458).  Here they stay resident in
their compressed form, in a per-layer (16,8) pool, and run through the same
two fused launches with the stage-2 codebook: a step whose experts mix both
kinds splits each token's pairs into a 2 bpw set on the paged pool and a
3 bpw set on the promoted pool (padded to a common width with weight-0 pairs
on an expert of the same step), and the second combine adds into the first's
output.
"""
from __future__ import annotations

import ctypes
import json
import os
import struct
from collections import OrderedDict

import torch

from . import kernels as K
from .rot import get_rot

MAGIC = b"VQ2M"
VERSION = 1
HEADER_FORMAT = "<4sHHHH QQQQQ 12s"
ENTRY_FORMAT = "<QIQIQIQI"
HEADER_SIZE = struct.calcsize(HEADER_FORMAT)
ENTRY_SIZE = struct.calcsize(ENTRY_FORMAT)


class Vq2mStore:
    """Reader of a ``.vq2m`` container (offset mode: no mapping of the file)."""

    def __init__(self, path):
        self.path = str(path)
        self.fd = os.open(self.path, os.O_RDONLY)
        head = os.pread(self.fd, HEADER_SIZE, 0)
        if len(head) != HEADER_SIZE:
            raise ValueError(f"{self.path}: truncated header")
        (magic, version, self.num_layers, self.num_experts, _, table_off, table_len, meta_off, meta_len,
         self.payload_start, _) = struct.unpack(HEADER_FORMAT, head)
        if magic != MAGIC or version != VERSION:
            raise ValueError(f"{self.path}: not a version-{VERSION} .vq2m container")
        if table_len != self.num_layers * self.num_experts * ENTRY_SIZE:
            raise ValueError(f"{self.path}: expert table of {table_len} bytes for "
                             f"{self.num_layers} x {self.num_experts} entries")
        table = os.pread(self.fd, table_len, table_off)
        entries = list(struct.iter_unpack(ENTRY_FORMAT, table))
        self.entries = [entries[l * self.num_experts:(l + 1) * self.num_experts] for l in range(self.num_layers)]
        self.meta = json.loads(os.pread(self.fd, meta_len, meta_off).decode("utf-8"))
        self.gu_rows = int(self.meta.get("gu_rows", 1024))
        self.gu_cols = int(self.meta.get("gu_cols", 256))
        self.dn_rows = int(self.meta.get("dn_rows", 2048))
        self.dn_cols = int(self.meta.get("dn_cols", 64))
        self.expert_modes = self.meta.get("expert_modes", {})
        # byte sizes of one 2 bpw record (index planes int16, scales fp16)
        self.sizes = (self.gu_rows * self.gu_cols * 2, self.gu_rows * 2, self.dn_rows * self.dn_cols * 2,
                      self.dn_rows * 2)
        self.record_bytes = sum(self.sizes)
        # promoted (16,8) record: int16 stage-1 plane followed by the uint8 stage-2 plane
        self.promoted_sizes = (self.gu_rows * self.gu_cols * 3, self.gu_rows * 2, self.dn_rows * self.dn_cols * 3,
                               self.dn_rows * 2)

    def promoted(self, layer: int, expert: int) -> bool:
        return self.expert_modes.get(f"{layer}:{expert}") == 3

    def promoted_experts(self, layer: int) -> list:
        return [e for e in range(self.num_experts) if self.promoted(layer, e)]

    def read_promoted(self, layer: int, expert: int) -> dict:
        """CPU tensors of a promoted expert: gu0 int16 / gu1 uint8 [gu_rows,
        gu_cols], gu_s fp16 [gu_rows], dn0 / dn1 [dn_rows, dn_cols], dn_s."""
        if not self.promoted(layer, expert):
            raise ValueError(f"layer {layer} expert {expert} is not a promoted 3-bit expert")
        e = self.entries[layer][expert]
        offs, szs = e[0::2], e[1::2]
        if tuple(szs) != self.promoted_sizes:
            raise ValueError(f"layer {layer} expert {expert}: record sizes {szs} are not a (16,8) expert "
                             f"{self.promoted_sizes}")
        parts = []
        for off, sz in zip(offs, szs):
            b = os.pread(self.fd, sz, off)
            if len(b) != sz:
                raise IOError(f"short read of layer {layer} expert {expert}")
            parts.append(torch.frombuffer(bytearray(b), dtype=torch.uint8))
        gi, gs, di, ds = parts
        a, b = self.gu_rows * self.gu_cols * 2, self.dn_rows * self.dn_cols * 2
        return {"gu0": gi[:a].view(torch.int16).view(self.gu_rows, self.gu_cols),
                "gu1": gi[a:].view(self.gu_rows, self.gu_cols),
                "gu_s": gs.view(torch.float16),
                "dn0": di[:b].view(torch.int16).view(self.dn_rows, self.dn_cols),
                "dn1": di[b:].view(self.dn_rows, self.dn_cols),
                "dn_s": ds.view(torch.float16)}

    def read_record(self, layer: int, expert: int, dst: memoryview) -> None:
        """Read the expert's [gate_up idx | gate_up scale | down idx | down
        scale] record into dst (record_bytes long)."""
        e = self.entries[layer][expert]
        offs, szs = e[0::2], e[1::2]
        if tuple(szs) != self.sizes:
            raise ValueError(f"layer {layer} expert {expert}: record sizes {szs} are not a 2 bpw expert {self.sizes}"
                             + (" (promoted 3-bit expert)" if self.promoted(layer, expert) else ""))
        contiguous = all(offs[i] + szs[i] == offs[i + 1] for i in range(3))
        if contiguous:
            got = os.preadv(self.fd, [dst[:self.record_bytes]], offs[0])
            if got != self.record_bytes:
                raise IOError(f"short read of layer {layer} expert {expert}")
            return
        pos = 0
        for off, sz in zip(offs, szs):
            if os.preadv(self.fd, [dst[pos:pos + sz]], off) != sz:
                raise IOError(f"short read of layer {layer} expert {expert}")
            pos += sz

    def close(self):
        if self.fd >= 0:
            os.close(self.fd)
            self.fd = -1

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write_vq2m(path, gate_up_idx, gate_up_scale, down_idx, down_scale, meta=None, payload_start=4096,
               promoted=None):
    """Write a container with the reference's layout: tensors per layer of
    shape [E, gu_rows, gu_cols] int16, [E, gu_rows] fp16, [E, dn_rows,
    dn_cols] int16, [E, dn_rows] fp16 (lists over layers, CPU tensors).
    promoted: {(layer, expert): (gu_idx1, dn_idx1)} uint8 stage-2 planes of
    3 bpw experts, written after their int16 planes in the index entries and
    flagged in meta["expert_modes"] (tools/build_mixed_b2_container.py)."""
    L = len(gate_up_idx)
    E, gu_rows, gu_cols = gate_up_idx[0].shape
    _, dn_rows, dn_cols = down_idx[0].shape
    promoted = dict(promoted or {})
    m = {"gu_rows": gu_rows, "gu_cols": gu_cols, "dn_rows": dn_rows, "dn_cols": dn_cols}
    m.update(meta or {})
    if promoted:
        m["expert_modes"] = {f"{l}:{e}": 3 for (l, e) in sorted(promoted)}
    meta_bytes = json.dumps(m).encode("utf-8")
    table_off = HEADER_SIZE
    table_len = L * E * ENTRY_SIZE
    meta_off = table_off + table_len
    start = max(payload_start, (meta_off + len(meta_bytes) + 4095) // 4096 * 4096)
    entries = []
    with open(path, "wb") as f:
        f.seek(start)
        for l in range(L):
            for e in range(E):
                ent = []
                s2 = promoted.get((l, e))
                for i, t in enumerate((gate_up_idx[l][e].to(torch.int16), gate_up_scale[l][e].to(torch.float16),
                                       down_idx[l][e].to(torch.int16), down_scale[l][e].to(torch.float16))):
                    b = t.contiguous().view(torch.uint8).numpy().tobytes()
                    if s2 is not None and i in (0, 2):
                        b += s2[i // 2].to(torch.uint8).contiguous().numpy().tobytes()
                    ent += [f.tell(), len(b)]
                    f.write(b)
                entries.append(struct.pack(ENTRY_FORMAT, *ent))
        f.seek(0)
        f.write(struct.pack(HEADER_FORMAT, MAGIC, VERSION, L, E, 0, table_off, table_len, meta_off, len(meta_bytes),
                            start, b"\0" * 12))
        f.write(b"".join(entries))
        f.write(meta_bytes)


class ExpertPager:
    """Device pool of `capacity` expert slots of one layer, filled from a
    Vq2mStore, LRU replacement (vq2/paged_runtime.py:415-437).

    ``device_tables=True`` (GPU only): the slot tables live on the device
    and each step is paged by two launches (vq2_pager_step, vq2_pager_copy)
    from a pinned host mirror of the layer's records, read from the file
    once here: no host synchronisation, so the step can be captured in a HIP
    graph.  The least recently used slot a step does not need is replaced,
    as on the host; an expert id outside the layer, or more distinct experts
    in a step than slots, gives NaN rows and sets ``errors`` (bit 1 / bit 2)
    instead of raising.

    ``sorted_layout=True`` (with device tables): the mirror holds every
    expert of the layer in the code-sorted layout (packed here once, all
    experts with the layer's common iteration counts) and the slots are a
    sorted pool (``sorted_gu`` / ``sorted_dn``) that the one-launch sorted
    MoE reads; the copy kernel moves a sorted record (~1.5x the bytes of a
    container record) per miss.  The reference-layout slot pools are not
    allocated then."""

    def __init__(self, store: Vq2mStore, layer: int, capacity: int, device, staging: int = 16,
                 scale_dtype=torch.bfloat16, device_tables: bool = False, sorted_layout: bool = False):
        self.store, self.layer, self.capacity = store, int(layer), int(capacity)
        self.device = torch.device(device)
        s = store
        sdt = scale_dtype or torch.float16
        self.sorted_layout = bool(sorted_layout)
        if self.sorted_layout and not device_tables:
            raise K.Vq2Error("the sorted slot pool is paged on the device: pass device_tables=True")
        if not self.sorted_layout:
            self.pool_gu_idx = torch.empty((capacity, s.gu_rows, s.gu_cols), dtype=torch.int16, device=self.device)
            self.pool_dn_idx = torch.empty((capacity, s.dn_rows, s.dn_cols), dtype=torch.int16, device=self.device)
        self.pool_gu_scale = torch.empty((capacity, s.gu_rows), dtype=sdt, device=self.device)
        self.pool_dn_scale = torch.empty((capacity, s.dn_rows), dtype=sdt, device=self.device)
        self.slot_of: OrderedDict[int, int] = OrderedDict()  # expert -> slot, least recently used first
        self.free = list(range(capacity - 1, -1, -1))
        self._hits = self._misses = 0
        cuda = self.device.type == "cuda"
        self.cuda = cuda
        self.device_tables = bool(device_tables)
        if self.device_tables:
            self._init_device_tables()
            return
        self.ring = [torch.empty(s.record_bytes, dtype=torch.uint8, pin_memory=cuda) for _ in range(staging)]
        self.ring_event = [None] * staging
        self.ring_pos = 0
        self.copy_stream = torch.cuda.Stream(device=self.device) if cuda else None

    # ------------------------------------------------------ device tables
    def _init_device_tables(self):
        s, dev = self.store, self.device
        if not self.cuda:
            raise K.Vq2Error("device_tables needs a GPU device")
        if any(sz % 16 for sz in s.sizes):
            raise K.Vq2Error(f"device_tables needs 16-byte record segments, got {s.sizes}")
        if s.promoted_experts(self.layer):
            raise K.Vq2Error(f"layer {self.layer} holds promoted 3-bit experts: use the host pager")
        E, C = s.num_experts, self.capacity
        if self.sorted_layout:
            self._init_sorted_mirror()
        else:
            self.mirror = torch.empty((E, s.record_bytes), dtype=torch.uint8, pin_memory=True)
            for e in range(E):
                s.read_record(self.layer, e, memoryview(self.mirror[e].numpy()))
            self._seg = (ctypes.c_int64 * 4)(*s.sizes)
            pools = (self.pool_gu_idx, self.pool_gu_scale, self.pool_dn_idx, self.pool_dn_scale)
        i32 = dict(dtype=torch.int32, device=dev)
        self.d_slot_of = torch.full((E,), -1, **i32)
        self.d_expert_of = torch.full((C,), -1, **i32)
        self.d_stamp = torch.full((C,), -1, **i32)
        self.d_state = torch.zeros(5, **i32)
        if self.sorted_layout:
            gw, dw = self.sorted_gu.expert_words() * 4, self.sorted_dn.expert_words() * 4
            self._dst = (ctypes.c_void_p * 4)(self.sorted_gu.entries.data_ptr(), self.pool_gu_scale.data_ptr(),
                                              self.sorted_dn.entries.data_ptr(), self.pool_dn_scale.data_ptr())
            self._dst_stride = (ctypes.c_int64 * 4)(gw, self.pool_gu_scale[0].numel() * self.pool_gu_scale.element_size(),
                                                    dw, self.pool_dn_scale[0].numel() * self.pool_dn_scale.element_size())
        else:
            self._dst = (ctypes.c_void_p * 4)(*[t.data_ptr() for t in pools])
            self._dst_stride = (ctypes.c_int64 * 4)(*[t[0].numel() * t.element_size() for t in pools])
        self._scale_dt = K._dt(self.pool_gu_scale, "scale")
        self._bufs = {}

    def _init_sorted_mirror(self):
        """Every expert of the layer in the code-sorted layout, in a pinned
        mirror of records [gate_up entries | gate_up fp16 scales | down
        entries | down fp16 scales], and the empty sorted slot pools."""
        s, E = self.store, self.store.num_experts
        raw = torch.empty((E, s.record_bytes), dtype=torch.uint8)
        for e in range(E):
            s.read_record(self.layer, e, memoryview(raw[e].numpy()))
        a, b, c = s.sizes[0], s.sizes[0] + s.sizes[1], s.sizes[0] + s.sizes[1] + s.sizes[2]
        gu = raw[:, :a].contiguous().view(torch.int16).view(E, s.gu_rows, s.gu_cols)
        dn = raw[:, b:c].contiguous().view(torch.int16).view(E, s.dn_rows, s.dn_cols)
        pgu = K.SortedPool(gu, device="cpu")
        pdn = K.SortedPool(dn, device="cpu")
        gw, dw = pgu.expert_words(), pdn.expert_words()
        sizes = (gw * 4, s.sizes[1], dw * 4, s.sizes[3])
        self._seg = (ctypes.c_int64 * 4)(*sizes)
        self.mirror_record_bytes = sum(sizes)
        self.mirror = torch.empty((E, self.mirror_record_bytes), dtype=torch.uint8, pin_memory=True)
        o1, o2, o3 = sizes[0], sizes[0] + sizes[1], sizes[0] + sizes[1] + sizes[2]
        self.mirror[:, :o1].copy_(pgu.entries.view(E, gw).view(torch.uint8).view(E, -1))
        self.mirror[:, o1:o2].copy_(raw[:, a:b])
        self.mirror[:, o2:o3].copy_(pdn.entries.view(E, dw).view(torch.uint8).view(E, -1))
        self.mirror[:, o3:].copy_(raw[:, c:])
        self.sorted_gu = K.SortedPool.slots(pgu, self.capacity, self.device)
        self.sorted_dn = K.SortedPool.slots(pdn, self.capacity, self.device)

    def step(self, ids):
        """Slots of a step's routed ids (device int32 / int64 [T, P]) ->
        device int32 [T, P], paged on the device (device_tables mode)."""
        if not self.device_tables:
            raise K.Vq2Error("step() pages on the device: construct with device_tables=True")
        ids = ids.contiguous()
        n = ids.numel()
        if ids.dtype not in (torch.int32, torch.int64) or ids.device != self.device:
            raise K.Vq2Error("ids must be int32 / int64 on the pool's device")
        if n not in self._bufs:
            self._bufs[n] = (torch.empty((n, 2), dtype=torch.int32, device=self.device),
                             torch.empty(n, dtype=torch.int32, device=self.device))
        copy_list, pair_slot = self._bufs[n]
        st = K._stream(self.device)
        i64 = 1 if ids.dtype == torch.int64 else 0
        E = self.store.num_experts
        K._lib.call("vq2_pager_step", ids.data_ptr(), i64, n, E, self.capacity, self.d_slot_of.data_ptr(),
                    self.d_expert_of.data_ptr(), self.d_stamp.data_ptr(), self.d_state.data_ptr(),
                    copy_list.data_ptr(), pair_slot.data_ptr(), st)
        rec = self.mirror_record_bytes if self.sorted_layout else self.store.record_bytes
        K._lib.call("vq2_pager_copy", self.mirror.data_ptr(), rec, self._seg,
                    copy_list.data_ptr(), self.d_state.data_ptr(), n, self._dst, self._dst_stride, self._scale_dt, st)
        return pair_slot.view(ids.shape)

    def _device_state(self):
        return self.d_state.cpu().tolist()

    @property
    def hits(self):
        return self._device_state()[2] if self.device_tables else self._hits

    @property
    def misses(self):
        return self._device_state()[3] if self.device_tables else self._misses

    @property
    def errors(self):
        """Device tables: bit 1 = an expert id outside the layer, bit 2 = more
        distinct experts in a step than slots (those pairs gave NaN)."""
        return self._device_state()[4] if self.device_tables else 0

    def _slot(self, expert: int, pending: list) -> int:
        if expert in self.slot_of:
            self._hits += 1
            self.slot_of.move_to_end(expert)
            return self.slot_of[expert]
        self._misses += 1
        # with at most `capacity` distinct experts per step the least recently
        # used resident expert is never one this step needs
        slot = self.free.pop() if self.free else self.slot_of.popitem(last=False)[1]
        self.slot_of[expert] = slot
        pending.append((expert, slot))
        return slot

    def ensure(self, experts) -> list:
        """Slots of `experts` (host ints), loading the missing ones; on a GPU
        the copies are queued and the current stream is made to wait for them.
        A request that cannot be served changes nothing; a failed read drops
        the experts it was loading from the pool."""
        if self.device_tables:
            raise K.Vq2Error("this pager keeps its tables on the device: use step()")
        ex = [int(e) for e in experts]
        for e in ex:
            if not 0 <= e < self.store.num_experts:
                raise K.Vq2Error(f"expert id {e} outside [0, {self.store.num_experts})")
        if len(set(ex)) > self.capacity:
            raise RuntimeError(f"{len(set(ex))} distinct experts in one step exceed the pool capacity {self.capacity}")
        pending: list = []
        slots = [self._slot(e, pending) for e in ex]
        if pending:
            try:
                self._load(pending)
            except BaseException:
                for e, slot in pending:
                    if self.slot_of.get(e) == slot:
                        del self.slot_of[e]
                        self.free.append(slot)
                raise
        return slots

    def _load(self, pending):
        s = self.store
        a, b, c = s.sizes[0], s.sizes[0] + s.sizes[1], s.sizes[0] + s.sizes[1] + s.sizes[2]
        if not self.cuda:
            for expert, slot in pending:
                buf = self.ring[0]
                s.read_record(self.layer, expert, memoryview(buf.numpy()))
                self._scatter(buf, slot, a, b, c)
            return
        compute = torch.cuda.current_stream(self.device)
        # slots being overwritten may still be read by launches already queued
        self.copy_stream.wait_stream(compute)
        for expert, slot in pending:
            i = self.ring_pos
            self.ring_pos = (i + 1) % len(self.ring)
            if self.ring_event[i] is not None:
                self.ring_event[i].synchronize()  # the staging record's previous copy
            buf = self.ring[i]
            s.read_record(self.layer, expert, memoryview(buf.numpy()))
            with torch.cuda.stream(self.copy_stream):
                self._scatter(buf, slot, a, b, c)
                ev = torch.cuda.Event()
                ev.record(self.copy_stream)
            self.ring_event[i] = ev
        compute.wait_stream(self.copy_stream)

    def _scatter(self, buf, slot, a, b, c):
        s = self.store
        nb = self.cuda
        self.pool_gu_idx[slot].copy_(buf[:a].view(torch.int16).view(s.gu_rows, s.gu_cols), non_blocking=nb)
        self.pool_gu_scale[slot].copy_(buf[a:b].view(torch.float16), non_blocking=nb)
        self.pool_dn_idx[slot].copy_(buf[b:c].view(torch.int16).view(s.dn_rows, s.dn_cols), non_blocking=nb)
        self.pool_dn_scale[slot].copy_(buf[c:].view(torch.float16), non_blocking=nb)


class PagedMoEExperts(torch.nn.Module):
    """Routed experts of one MoE layer over a paged device pool:
    forward(hidden_states [T, H], topk_idx [T, K], topk_weights [T, K]) ->
    [T, H] (vq2/paged_runtime.py:439-568, T == 1 fast path 491-511).
    cb8 is the [256, 8] stage-2 codebook of the (16,8) scheme, needed when
    the layer holds promoted 3 bpw experts."""

    def __init__(self, layer: int, store: Vq2mStore, cb16, capacity: int = 96, device="cuda", staging: int = 16,
                 act_dtype=torch.float32, out_dtype=None, cb8=None, scale_dtype=torch.bfloat16,
                 device_tables: bool = False, sorted_layout=None):
        super().__init__()
        dev = torch.device(device)
        H, I = store.gu_cols * 8, store.dn_cols * 8
        if sorted_layout is None:  # the device pager over a sorted slot pool where the sorted MoE runs
            sorted_layout = (device_tables and dev.type == "cuda" and act_dtype == torch.float32
                             and cb16.dtype in (torch.float16, torch.bfloat16) and H % 64 == 0 and I % 64 == 0
                             and H <= 8192 and I <= 8192 and not store.promoted_experts(layer))
        self.pager = ExpertPager(store, layer, capacity, device, staging, scale_dtype, device_tables,
                                 sorted_layout=bool(sorted_layout))
        self.cb16 = cb16
        self.hidden_dim = H
        self.intermediate_dim = I
        if store.gu_rows != 2 * self.intermediate_dim or store.dn_rows != self.hidden_dim:
            raise K.Vq2Error("inconsistent gate_up / down shapes in the container")
        self.rot_h = get_rot("moe_expert_2048", self.hidden_dim, dev)
        self.rot_i = get_rot("moe_expert_512", self.intermediate_dim, dev)
        self.act_dtype = act_dtype
        self.out_dtype = out_dtype
        # promoted (16,8) experts of this layer: resident, compressed
        promoted = store.promoted_experts(layer)
        self.promoted_index = {e: i for i, e in enumerate(promoted)}
        self.cb8 = None
        if promoted:
            if cb8 is None:
                raise K.Vq2Error(f"layer {layer} holds promoted 3-bit experts {promoted}: pass cb8, the [256, 8] "
                                 "stage-2 codebook")
            recs = [store.read_promoted(layer, e) for e in promoted]
            self.pro = {k: torch.stack([r[k] for r in recs]).to(dev) for k in recs[0]}
            if scale_dtype is not None:
                for k in ("gu_s", "dn_s"):
                    self.pro[k] = self.pro[k].to(scale_dtype)
            self.cb8 = cb8
            # the promoted pool also in the two-stage sorted layout, where the
            # one-launch sorted MoE runs (stage-2 codes into cb8)
            self.pro_sorted = None
            if (dev.type == "cuda" and act_dtype == torch.float32 and cb16.dtype in (torch.float16, torch.bfloat16)
                    and cb8.dtype == cb16.dtype and self.hidden_dim % 64 == 0 and self.intermediate_dim % 64 == 0):
                self.pro_sorted = (K.SortedPool(self.pro["gu0"], device=dev, idx1=self.pro["gu1"]),
                                   K.SortedPool(self.pro["dn0"], device=dev, idx1=self.pro["dn1"]))

    def _run(self, h, ids_d, w_d, pool, accumulate_into=None):
        """Two launches over one pool: gate_up with the H-point RHT, then
        SwiGLU + I-point RHT + down + weighted combine (out= / out+=)."""
        T, P = ids_d.shape
        I = self.intermediate_dim
        y_gu = torch.empty((T * P, 2 * I), dtype=self.act_dtype, device=h.device)
        gu0, gu1, gus, dn0, dn1, dns = pool
        cb8 = self.cb8 if gu1 is not None else None
        K.vq_moe_gate_up_rht(h, ids_d, gu0, self.cb16, gus, y_gu, OUT=2 * I, NG=self.hidden_dim // 8,
                             perm=self.rot_h._perm32, sign=self.rot_h._sign8, hb=self.rot_h.hb,
                             rht_scale=self.rot_h.scale, pool1=gu1, cb8=cb8)
        return K.vq_moe_down_swiglu_combine(y_gu, ids_d, w_d, dn0, self.cb16, dns, OUT=self.hidden_dim, NG=I // 8,
                                            perm=self.rot_i._perm32, sign=self.rot_i._sign8, hb=self.rot_i.hb,
                                            rht_scale=self.rot_i.scale, out=accumulate_into,
                                            out_dtype=torch.float32, pool1=dn1, cb8=cb8,
                                            accumulate=accumulate_into is not None)

    def _table(self, rows, dev):
        """Device tensors of a padded [T, width] pair table: pool ids (int32),
        source columns into topk_weights (int64) and a 0/1 weight mask.
        rows[t] = [(pool id, column), ...]; a padding pair repeats the
        table's first pool id with weight 0."""
        width = max(len(r) for r in rows)
        pad = next(r[0][0] for r in rows if r)
        ids = [[r[j][0] if j < len(r) else pad for j in range(width)] for r in rows]
        cols = [[r[j][1] if j < len(r) else 0 for j in range(width)] for r in rows]
        mask = [[1.0 if j < len(r) else 0.0 for j in range(width)] for r in rows]
        pin = dev.type == "cuda"
        to = lambda v, dt: torch.tensor(v, dtype=dt, pin_memory=pin).to(dev, non_blocking=True)
        return to(ids, torch.int32), to(cols, torch.int64), to(mask, torch.float32)

    def forward(self, hidden_states, topk_idx, topk_weights):
        p = self.pager
        h = hidden_states.reshape(-1, self.hidden_dim).contiguous()
        T = h.shape[0]
        if p.device_tables:
            # paged on the device: no host synchronisation (graph-capturable)
            ids_d = topk_idx.reshape(T, -1)
            if ids_d.dtype not in (torch.int32, torch.int64):
                ids_d = ids_d.to(torch.int32)
            P = ids_d.shape[1]
            w = topk_weights.reshape(T, P).to(device=h.device, dtype=torch.float32).contiguous()
            slots = p.step(ids_d.to(h.device))
            if p.sorted_layout:
                rh, ri = self.rot_h, self.rot_i
                out = K.vq_sorted_moe(h, p.sorted_gu, p.pool_gu_scale, p.sorted_dn, p.pool_dn_scale, self.cb16,
                                      (rh._perm32, rh._sign8, rh.hb, rh.scale), (ri._perm32, ri._sign8, ri.hb, ri.scale),
                                      ids=slots, w=w)
                return out.to(self.out_dtype or hidden_states.dtype)
            regular = (p.pool_gu_idx, None, p.pool_gu_scale, p.pool_dn_idx, None, p.pool_dn_scale)
            return self._run(h, slots, w, regular).to(self.out_dtype or hidden_states.dtype)
        ids_host = topk_idx.reshape(T, -1).to("cpu")  # the paging decision is made on the host
        P = ids_host.shape[1]
        w = topk_weights.reshape(T, P).to(device=h.device, dtype=torch.float32).contiguous()
        regular = (p.pool_gu_idx, None, p.pool_gu_scale, p.pool_dn_idx, None, p.pool_dn_scale)
        flat = ids_host.reshape(-1).tolist()
        if not any(e in self.promoted_index for e in flat):
            slots = p.ensure(flat)
            slot_t = torch.tensor(slots, dtype=torch.int32, pin_memory=p.cuda).view(T, P)
            out = self._run(h, slot_t.to(h.device, non_blocking=True), w, regular)
            return out.to(self.out_dtype or hidden_states.dtype)
        # mixed step: 2 bpw pairs on the paged pool, promoted pairs on the (16,8) pool
        rows = ids_host.tolist()
        reg = [[(e, j) for j, e in enumerate(r) if e not in self.promoted_index] for r in rows]
        pro = [[(self.promoted_index[e], j) for j, e in enumerate(r) if e in self.promoted_index] for r in rows]
        out = None
        if any(reg):
            slots = iter(p.ensure([e for r in reg for e, _ in r]))
            reg = [[(next(slots), j) for _, j in r] for r in reg]
            ids_d, cols_d, mask_d = self._table(reg, h.device)
            out = self._run(h, ids_d, torch.gather(w, 1, cols_d) * mask_d, regular)
        ids_d, cols_d, mask_d = self._table(pro, h.device)
        pp = self.pro
        wp = torch.gather(w, 1, cols_d) * mask_d
        if self.pro_sorted is not None:
            # promoted pairs on the sorted two-stage pool, added to the 2 bpw
            # pairs' sum (per token: 2 bpw pairs, then promoted pairs)
            rh, ri = self.rot_h, self.rot_i
            out_p = K.vq_sorted_moe(h, self.pro_sorted[0], pp["gu_s"], self.pro_sorted[1], pp["dn_s"], self.cb16,
                                    (rh._perm32, rh._sign8, rh.hb, rh.scale), (ri._perm32, ri._sign8, ri.hb, ri.scale),
                                    ids=ids_d, w=wp, cb1=self.cb8)
            out = out_p if out is None else out + out_p
        else:
            out = self._run(h, ids_d, wp, (pp["gu0"], pp["gu1"], pp["gu_s"], pp["dn0"], pp["dn1"], pp["dn_s"]),
                            accumulate_into=out)
        return out.to(self.out_dtype or hidden_states.dtype)
