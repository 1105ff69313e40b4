#!/usr/bin/env python
"""Benchmark of the VQ2 decode hot path on one MI355X.

Headline: one decoder layer's projection set at
batch 1, hidden 2048 -- RHT(2048) -> q, k, v (2 bpw); RHT(2048) -> o (2 bpw);
RHT(2048) -> gate, up (4 bpw, two 16-bit stages); RHT(6144, 3 x 2048 blocks)
-> down (4 bpw), as four launches that each rotate their activation in LDS.
One step = one layer; the timed loop cycles through L
distinct layer weight sets (>= 1 GiB in total) so the 256 MB Infinity Cache
cannot hold the weights, and replays the launches as HIP graphs.
``value`` = compressed weight bytes (index planes + row scales) per step /
step time, in GB/s.

Also reported: the config-4 MoE layer (router + 8 routed + 1 shared expert,
T = 1) in us per layer over a 40-layer resident pool, the config-3 LM head
(151936 x 2048, 2 bpw, fused top-1), the dominant kernel's roofline
(4 bpw GEMV, HIP events on its stream) and the reference CPU path timed on
the host (``cpu_baseline``).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
                       [--only dominant|dominant_gather|dense|copy|moe|paged] (single-part modes for rocprofv3 runs)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0  # dense fp16 matrix-core peak of MI355X
HIDDEN, Q_OUT, KV_OUT, INTER = 2048, 2048, 512, 6144


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def metric_name() -> str:
    try:
        return json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    except Exception:
        return "VQ-GEMV HBM GB/s (% of peak) + us per 35B-A3B-shape MoE layer at batch 1"


# ----------------------------------------------------------------- workloads
def rand_i16(shape, g, dev):
    import torch

    return torch.randint(-32768, 32768, shape, generator=g, device=dev, dtype=torch.int32).to(torch.int16)


def rand_scale(n, g, dev):
    import torch

    return (torch.rand(n, generator=g, device=dev) + 0.5).to(torch.float16)


class DenseLayers:
    """L layer sets of the configs[1] projections (device-resident).  As
    PackedLinear does, the large matrices (gate, up, down: >= 2M codes) also
    get the code-sorted layout, packed once here, and so do q, k and v, which
    PackedProjections runs in one launch (0.79 M codes together)."""

    PROJ = [  # name, out, n, bpw
        ("q", Q_OUT, HIDDEN, 2), ("k", KV_OUT, HIDDEN, 2), ("v", KV_OUT, HIDDEN, 2), ("o", HIDDEN, HIDDEN, 2),
        ("gate", INTER, HIDDEN, 4), ("up", INTER, HIDDEN, 4), ("down", HIDDEN, INTER, 4),
    ]

    def __init__(self, L, dev):
        import torch

        from compressai_amd import kernels as K, synth
        from compressai_amd.runtime import SORTED_MIN_CODES, SORTED_MIN_LAUNCH_CODES

        self.L, self.dev = L, dev
        g = torch.Generator(device=dev).manual_seed(2000)
        self.cb0 = synth.codebook(2000).to(dev)
        self.cb1 = synth.codebook(2001).to(dev)
        self.layers = []
        t0 = time.perf_counter()
        qkv_codes = sum(out * (n // 8) * (2 if bpw == 4 else 1) for name, out, n, bpw in self.PROJ[:3])
        # q, k and v share one chunk height over their rows, as PackedProjections packs them
        qkv_R = K.sorted_launch_rows_per_chunk([out for _, out, _, _ in self.PROJ[:3]], HIDDEN // 8, dev)
        for _ in range(L):
            lay = {}
            for name, out, n, bpw in self.PROJ:
                i0 = rand_i16((out, n // 8), g, dev)
                i1 = rand_i16((out, n // 8), g, dev) if bpw == 4 else None
                sp = None
                codes = out * (n // 8) * (2 if bpw == 4 else 1)
                if name in ("q", "k", "v") and qkv_codes >= SORTED_MIN_LAUNCH_CODES:
                    sp = K.SortedPlanes(i0, i1, out, n, device=dev, rows_per_chunk=qkv_R)
                elif codes >= SORTED_MIN_CODES:
                    sp = K.SortedPlanes(i0, i1, out, n, device=dev)
                lay[name] = (i0, i1, rand_scale(out, g, dev), out, n, sp)
            self.layers.append(lay)
        log(f"dense: {L} layer sets generated, large matrices packed to the sorted layout in "
            f"{time.perf_counter() - t0:.1f} s")
        self.bytes_per_step = sum(out * (n // 8) * 2 * (2 if bpw == 4 else 1) + out * 2
                                  for _, out, n, bpw in self.PROJ)
        # resident index bytes of one layer set: the reference planes, and the
        # code-sorted copies kept beside them
        lay0 = self.layers[0]
        self.plane_bytes = sum(t.numel() * t.element_size() for v in lay0.values() for t in v[:2] if t is not None)
        self.sorted_bytes = sum(v[5].nbytes() for v in lay0.values() if v[5] is not None)
        self.x_attn = synth.activations(2004, HIDDEN).to(dev)
        self.x_o = synth.activations(2014, HIDDEN).to(dev)
        self.x_mlp = synth.activations(2024, HIDDEN).to(dev)
        self.x_down = synth.activations(2034, INTER).to(dev)
        # the reference's rotation always permutes before the sign flip
        self.sign_h = synth.signs(2005, HIDDEN).to(dev)
        self.sign_i = synth.signs(2015, INTER).to(dev)
        self.perm_h = synth.permutation(2006, HIDDEN).to(dev)
        self.perm_i = synth.permutation(2016, INTER).to(dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.y = {name: torch.empty(out, **f32) for name, out, _, _ in self.PROJ}

    def fused(self, lay, names, x, perm, sign):
        """One gather-kernel launch: RHT of x built in LDS + the GEMVs of `names`."""
        from compressai_amd import kernels as K

        mats = [(lay[nm][0], lay[nm][1], lay[nm][2], lay[nm][3]) for nm in names]
        n = lay[names[0]][4]
        K.vq_gemv_rht(x, mats, self.cb0, self.cb1 if mats[0][1] is not None else None, n, perm, sign, 2048,
                      ys=[self.y[nm] for nm in names])

    def sorted(self, lay, names, x, perm, sign):
        """Sorted-layout launch: RHT built in LDS, slices summed in the launch."""
        from compressai_amd import kernels as K

        n = lay[names[0]][4]
        K.vq_sorted_gemv(x, [(lay[nm][5], lay[nm][2]) for nm in names], self.cb0,
                         self.cb1 if lay[names[0]][1] is not None else None, n, perm, sign, 2048,
                         ys=[self.y[nm] for nm in names])

    def step(self, l):
        """One decoder layer's projections, as the runtime runs them at batch
        1: q/k/v in one sorted-layout launch (PackedProjections), o, gate/up
        and down on the sorted layout (PackedLinear); every launch rotates its
        activation in LDS."""
        lay = self.layers[l]
        self.sorted(lay, ("q", "k", "v"), self.x_attn, self.perm_h, self.sign_h)
        self.sorted(lay, ("o",), self.x_o, self.perm_h, self.sign_h)
        self.sorted(lay, ("gate", "up"), self.x_mlp, self.perm_h, self.sign_h)
        self.sorted(lay, ("down",), self.x_down, self.perm_i, self.sign_i)

    def step_gather(self, l):
        """The same step with every matrix on the gather kernel (reference layout only)."""
        lay = self.layers[l]
        self.fused(lay, ("q", "k", "v"), self.x_attn, self.perm_h, self.sign_h)
        self.fused(lay, ("o",), self.x_o, self.perm_h, self.sign_h)
        self.fused(lay, ("gate", "up"), self.x_mlp, self.perm_h, self.sign_h)
        self.fused(lay, ("down",), self.x_down, self.perm_i, self.sign_i)


def capture(fn, n_items, dev):
    """HIP graph of fn(0..n_items-1) launched back to back."""
    import torch

    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for i in range(n_items):  # eager warm-up of every launch shape
            fn(i)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_items):
            fn(i)
    torch.cuda.synchronize(dev)
    return g


def time_graph(g, reps, dev):
    """(elapsed ms on the replay stream measured by HIP events, host ms)."""
    import torch

    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize(dev)
    return e0.elapsed_time(e1), (time.perf_counter() - t0) * 1e3


def time_steps(g_full, L, g_rest, steps, dev):
    """Replay exactly `steps` layer steps: steps // L replays of the L-layer
    graph, then the graph of the first steps % L layers.  Returns (ms, host ms)."""
    import torch

    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(steps // L):
        g_full.replay()
    if steps % L:
        g_rest.replay()
    e1.record(st)
    torch.cuda.synchronize(dev)
    return e0.elapsed_time(e1), (time.perf_counter() - t0) * 1e3


REPEATS = 5  # timed repetitions; the bench line reports their median


def bench_dense(args, dev):
    import torch

    L = args.layers
    dl = DenseLayers(L, dev)
    log(f"dense: {L} layer sets, {dl.bytes_per_step * L / 2**30:.2f} GiB of compressed weights")
    g = capture(dl.step, L, dev)
    rest = args.steps % L
    g_rest = capture(dl.step, rest, dev) if rest else None
    time_graph(g, max(1, -(-args.warmup // L)), dev)  # warm-up: at least W steps
    runs = [time_steps(g, L, g_rest, args.steps, dev) for _ in range(REPEATS)]
    per_step = sorted(ms / args.steps for ms, _ in runs)
    ms_per_step = statistics.median(per_step)
    host_ms = statistics.median(h for _, h in runs)
    gbps = dl.bytes_per_step / (ms_per_step * 1e-3) / 1e9
    log(f"dense: {args.steps} steps x {REPEATS} repetitions, median {ms_per_step * 1e3:.2f} us/step "
        f"(min {per_step[0] * 1e3:.2f}, max {per_step[-1] * 1e3:.2f}; host {host_ms:.3f} ms per repetition) -> "
        f"{gbps:.1f} GB/s")

    # the same step on the gather kernel only (reference layout)
    gg = capture(dl.step_gather, L, dev)
    time_graph(gg, 1, dev)
    gather_us = statistics.median(time_graph(gg, max(1, args.steps // L), dev)[0] * 1e3 / (max(1, args.steps // L) * L)
                                  for _ in range(REPEATS))
    del gg
    log(f"dense, gather kernel only: {gather_us:.2f} us/step, "
        f"{dl.bytes_per_step / (gather_us * 1e-6) / 1e9:.1f} GB/s")

    # dominant launch: gate + up (RHT + two 6144 x 2048 4 bpw matrices) on the
    # sorted layout (one launch, slices summed by the last workgroup), back to back
    # over the layer sets on the replay stream; also the gather-kernel launch
    dom_bytes = 2 * (INTER * (HIDDEN // 8) * 2 * 2 + INTER * 2)
    res = {}
    for name, fn in (("sorted", dl.sorted), ("gather", dl.fused)):
        gd = capture(lambda l, fn=fn: fn(dl.layers[l], ("gate", "up"), dl.x_mlp, dl.perm_h, dl.sign_h), L, dev)
        time_graph(gd, 2, dev)
        dreps = max(4, 2000 // L)
        res[name] = statistics.median(time_graph(gd, dreps, dev)[0] * 1e3 / (dreps * L) for _ in range(REPEATS))
        del gd
        log(f"gate+up launch ({name}): {res[name]:.2f} us/call, {dom_bytes / (res[name] * 1e-6) / 1e9:.1f} GB/s")
    dom_us = res["sorted"]
    dom_gbps = dom_bytes / (dom_us * 1e-6) / 1e9
    return dict(steps=args.steps, ms_per_step=ms_per_step, gbps=gbps, bytes_per_step=dl.bytes_per_step, layers=L,
                plane_bytes=dl.plane_bytes, sorted_bytes=dl.sorted_bytes,
                dom_us=dom_us, dom_gbps=dom_gbps, dom_bytes=dom_bytes, host_ms=host_ms, dense=dl,
                spread_us=[round(per_step[0] * 1e3, 3), round(per_step[-1] * 1e3, 3)],
                gather_step_us=gather_us, dom_gather_us=res["gather"])


def bench_config0(args, dev, copies=1024):
    """RHT(2048, permutation + signs) + 2 bpw GEMV 2048 x 2048 at
    batch 1, one fused launch per call, over 1024 distinct matrices (1 GiB):
    as PackedLinear runs it (code-sorted layout, about 0.75 x CUs chunks of
    one workgroup each), and on the gather kernel (vq_gemv_rht) beside it."""
    import torch

    from compressai_amd import kernels as K, synth

    n = out = 2048
    g = torch.Generator(device=dev).manual_seed(1000)
    cb = synth.codebook(1000).to(dev)
    mats = [(rand_i16((out, n // 8), g, dev), rand_scale(out, g, dev)) for _ in range(copies)]
    sps = [K.SortedPlanes(i0, None, out, n, device=dev) for i0, _ in mats]
    x = synth.activations(1004, n, dtype=torch.float16).to(dev)
    sign = synth.signs(1005, n).to(dev)
    perm = synth.permutation(1006, n).to(dev)
    y = torch.empty(out, dtype=torch.float32, device=dev)

    def fwd(l):
        K.vq_sorted_gemv(x, [(sps[l], mats[l][1])], cb, None, n, perm, sign, 2048, ys=[y])

    def fwd_gather(l):
        i0, s = mats[l]
        K.vq_gemv_rht(x, [(i0, None, s, out)], cb, None, n, perm, sign, 2048, ys=[y])

    res = {}
    for name, f in (("sorted", fwd), ("gather", fwd_gather)):
        gr = capture(f, copies, dev)
        time_graph(gr, 1, dev)
        res[name] = statistics.median(time_graph(gr, 1, dev)[0] * 1e3 / copies for _ in range(REPEATS))
        del gr
    us = res["sorted"]
    nbytes = out * (n // 8) * 2 + out * 2
    gbps = nbytes / (us * 1e-6) / 1e9
    log(f"config 0 (RHT 2048 + 2 bpw 2048x2048, {copies} copies): {us:.2f} us/call, {gbps:.1f} GB/s "
        f"({sps[0].n_chunks} chunks of {sps[0].rows_per_chunk} rows; gather kernel {res['gather']:.2f} us)")
    del mats, sps
    torch.cuda.empty_cache()
    return {"us": round(us, 3), "gbps": round(gbps, 2), "bytes": nbytes, "copies": copies,
            "us_gather_kernel": round(res["gather"], 3)}


def bench_moe(args, dev, n_layers=40, tokens=(1, 8)):
    """MoE layers over a 40-layer resident pool, T tokens per step
    for each T in `tokens` (the same pool, per-layer seeded router logits)."""
    import torch

    from compressai_amd import synth
    from compressai_amd.moe import MoELayer

    E, k = 256, 8
    g = torch.Generator(device=dev).manual_seed(4000)
    cb = synth.codebook(4000).to(dev)
    layers = []
    for _ in range(n_layers):
        gu = rand_i16((E + 1, 1024, 256), g, dev)
        gus = rand_scale((E + 1) * 1024, g, dev).view(E + 1, 1024)
        dn = rand_i16((E + 1, 2048, 64), g, dev)
        dns = rand_scale((E + 1) * 2048, g, dev).view(E + 1, 2048)
        gate = (torch.randn(HIDDEN, generator=g, device=dev) * 0.02).to(torch.float16)
        layers.append(MoELayer(gu, gus, dn, dns, cb, gate, top_k=k))
    per_expert = 1024 * 256 * 2 + 1024 * 2 + 2048 * 64 * 2 + 2048 * 2
    log(f"moe: {n_layers} layers x {E + 1} experts resident ({n_layers * (E + 1) * per_expert / 2**30:.2f} GiB)")
    res = {}
    for T in tokens:
        inputs = []
        for _ in range(n_layers):
            h = torch.randn(T, HIDDEN, generator=g, device=dev).to(torch.float16)
            lg = torch.randn(T, E, generator=g, device=dev).to(torch.float16)
            inputs.append((h, lg))
        outs = [None] * n_layers

        def fwd(l, inputs=inputs, outs=outs):
            outs[l] = layers[l](*inputs[l])

        gr = capture(fwd, n_layers, dev)
        time_graph(gr, 3, dev)
        reps = max(5, args.steps // n_layers)
        us = statistics.median(time_graph(gr, reps, dev)[0] * 1e3 / (reps * n_layers) for _ in range(REPEATS))
        # distinct experts actually read per layer (routed + shared)
        distinct = []
        for l in range(n_layers):
            ids, _ = layers[l].route(inputs[l][0], inputs[l][1])
            distinct.append(len(set(ids.flatten().tolist())))
        bytes_layer = statistics.mean(distinct) * per_expert
        gbps = bytes_layer / (us * 1e-6) / 1e9
        log(f"moe T={T}: {us:.2f} us/layer, {gbps:.1f} GB/s ({statistics.mean(distinct):.1f} experts/layer)")
        res[T] = dict(us=us, gbps=gbps, bytes=bytes_layer, cpu_inputs=inputs[0])
        del gr
    res["cpu_layer"] = layers[0]
    m0 = layers[0].experts_mod
    res["resident"] = dict(
        planes=sum(t.numel() * t.element_size() for t in (m0.gate_up_idx, m0.down_idx)),
        sorted=sum(p.nbytes() for p in (m0.sorted_gu, m0.sorted_dn, m0.sorted_dn_tall) if p is not None))
    return res


def bench_lm_head(args, dev, batch=1, copies=14, only=False):
    """LM head 151936 x 2048 at 2 bpw + top-1 over 14 copies
    (1.1 GiB).  Batch 1: the sorted layout with the RHT of the fp16
    activation built in the kernel (as PackedLMHead.argmax runs it), the
    same on a pre-rotated activation, and the gather kernel (pre-rotated);
    batch 4: the sorted batch kernel (pre-rotated, as PackedLMHead.argmax runs
    it after the RHT) and the matrix-core path."""
    import torch

    from compressai_amd import kernels as K, synth

    out, n = 151936, 2048
    g = torch.Generator(device=dev).manual_seed(3000)
    cb = synth.codebook(3000).to(dev)
    mats = []
    for _ in range(copies):
        i0, s = rand_i16((out, n // 8), g, dev), rand_scale(out, g, dev)
        mats.append((i0, s, K.SortedPlanes(i0, None, out, n, device=dev)))
    x = synth.activations(3004, (batch, n), dtype=torch.float32).to(dev)
    xh = synth.activations(3005, (batch, n), dtype=torch.float16).to(dev)
    perm, sign = synth.permutation(3006, n).to(dev), synth.signs(3007, n).to(dev)
    ws = torch.empty(batch, out, dtype=torch.float32, device=dev)
    res = [None] * copies
    nbytes = out * (n // 8) * 2 + out * 2

    if only:  # one call per copy, as the B = 1 runtime path runs it (for counter runs)
        for l in range(copies):
            _, s, sp = mats[l]
            K.vq_sorted_gemv_argmax(xh, sp, s, cb, None, n, perm, sign, 2048)
        torch.cuda.synchronize(dev)
        return None

    def run(fwd):
        gr = capture(fwd, copies, dev)
        time_graph(gr, 2, dev)
        reps = max(5, 200 // copies)
        us = statistics.median(time_graph(gr, reps, dev)[0] * 1e3 / (reps * copies) for _ in range(REPEATS))
        del gr
        return us

    def f_gather(l):
        i0, s, _ = mats[l]
        res[l] = K.vq_gemv_argmax(x, i0, None, cb, None, s, out, n, logits_ws=ws)

    def f_sorted(l):
        _, s, sp = mats[l]
        res[l] = K.vq_sorted_gemv_argmax(x, sp, s, cb, None, n)

    def f_sorted_rht(l):
        _, s, sp = mats[l]
        res[l] = K.vq_sorted_gemv_argmax(xh, sp, s, cb, None, n, perm, sign, 2048)

    def f_sorted_batch(l):
        _, s, sp = mats[l]
        res[l] = K.vq_sorted_gemm_batch_argmax(x, sp, s, cb, None, n)

    out_d = {}
    if batch == 1:
        us = run(f_sorted_rht)
        out_d["prerotated_us"] = run(f_sorted)
        out_d["gather_us"] = run(f_gather)
        log(f"lm head B=1 (sorted layout, pre-rotated x): {out_d['prerotated_us']:.2f} us/call")
        log(f"lm head B=1 (gather kernel, pre-rotated x): {out_d['gather_us']:.2f} us/call")
    else:
        us = run(f_sorted_batch)
        out_d["matrix_cores_us"] = run(f_gather)
        log(f"lm head B={batch} (matrix cores, pre-rotated x): {out_d['matrix_cores_us']:.2f} us/call")
    gbps = nbytes / (us * 1e-6) / 1e9
    log(f"lm head B={batch}: {us:.2f} us/call, {gbps:.1f} GB/s")
    out_d.update(us=us, gbps=gbps, plane_bytes=mats[0][0].numel() * 2, sorted_bytes=mats[0][2].nbytes())
    return out_d


def bench_small_m(args, dev):
    """small-M batched VQ GEMM on the matrix cores (M = 16, 64) on
    the 6144x2048 and 2048x6144 MLP shapes at 2 and 4 bpw, >= 1 GiB of
    distinct weights cycled; plus the RHT of the [M, 8192] activation (2048-
    point blocks as the reference's Rot picks for n = 8192, and one 8192-point
    block)."""
    import torch

    from compressai_amd import kernels as K, synth

    g = torch.Generator(device=dev).manual_seed(5000)
    cb0 = synth.codebook(5000).to(dev)
    cb1 = synth.codebook(5001).to(dev)
    res = {}
    for out, n in ((6144, 2048), (2048, 6144)):
        for bpw in (2, 4):
            per = out * (n // 8) * 2 * (2 if bpw == 4 else 1) + out * 2
            copies = int(2**30 // per) + 1
            mats = [(rand_i16((out, n // 8), g, dev), rand_i16((out, n // 8), g, dev) if bpw == 4 else None,
                     rand_scale(out, g, dev)) for _ in range(copies)]
            c1 = cb1 if bpw == 4 else None
            for M in (16, 64):
                x = synth.activations(5004 + M, (M, n), dtype=torch.float16).to(dev)
                y = torch.empty((M, out), dtype=torch.float32, device=dev)

                def fwd(l, x=x, y=y, c1=c1):
                    i0, i1, s = mats[l]
                    K.vq_gemm_small_m(x, i0, i1, cb0, c1, s, out, n, y=y)

                gr = capture(fwd, copies, dev)
                time_graph(gr, 1, dev)
                reps = max(2, 400 // copies)
                ms, _ = time_graph(gr, reps, dev)
                us = ms * 1e3 / (reps * copies)
                key = f"{out}x{n}_{bpw}bpw_M{M}"
                tflops = 2.0 * M * out * n / (us * 1e-6) / 1e12
                res[key] = {"us": round(us, 3), "gbps": round(per / (us * 1e-6) / 1e9, 2),
                            "tflops": round(tflops, 2), "mfma_frac": round(tflops / PEAK_MFMA_F16_TFLOPS, 5)}
                log(f"small-M {key}: {us:.2f} us/call, {res[key]['gbps']:.1f} GB/s, {tflops:.1f} TFLOP/s "
                    f"({100 * tflops / PEAK_MFMA_F16_TFLOPS:.2f} % of the fp16 MFMA peak)")
            del mats
            torch.cuda.empty_cache()
    sign = synth.signs(5006, 8192).to(dev)
    perm = synth.permutation(5008, 8192).to(dev)
    for M in (16, 64):
        x = synth.activations(5007, (M, 8192), dtype=torch.float16).to(dev)
        xr = torch.empty((M, 8192), dtype=torch.float32, device=dev)
        for hb in (2048, 8192):
            gr = capture(lambda l, x=x, hb=hb: K.vq_rht(x, perm, sign, hb, out=xr), 50, dev)
            time_graph(gr, 1, dev)
            ms, _ = time_graph(gr, 10, dev)
            us = ms * 1e3 / 500
            res[f"rht8192_hb{hb}_M{M}"] = {"us": round(us, 3)}
            log(f"RHT [M={M}, 8192] hb={hb}: {us:.2f} us/call")
    return res


def bench_unpack(args, dev):
    """Container load: fixed-width packed index streams -> int16 planes
    (vq2/export.py:56-70), 2^25 symbols per call; GB/s counts bytes read +
    written."""
    import torch

    from compressai_amd import kernels as K

    n = 1 << 25
    g = torch.Generator(device=dev).manual_seed(6000)
    res = {}
    for bits in (12, 16):
        nb = (n * bits + 7) // 8
        buf = torch.randint(0, 256, (nb,), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
        out = torch.empty(n, dtype=torch.int16, device=dev)
        gr = capture(lambda l: K.vq_unpack_fixed(buf, bits, n, out=out), 10, dev)
        time_graph(gr, 1, dev)
        ms, _ = time_graph(gr, 10, dev)
        us = ms * 1e3 / 100
        res[f"{bits}bit"] = {"us": round(us, 3), "gbps": round((nb + 2 * n) / (us * 1e-6) / 1e9, 1)}
        log(f"unpack_fixed {bits}-bit, {n} symbols: {us:.2f} us, {res[f'{bits}bit']['gbps']:.0f} GB/s")
    return res


def bench_paged(args, dev, E=64, steps=200):
    """Paged expert pool (config-4 expert shape, one layer of E experts in a
    .vq2m file): T = 1, top-8 routed ids on the device each step.  Warm: every
    expert resident; churn: 16 slots, so most steps page experts in.  Host
    pager: misses read from the file through the pinned ring, host-timed (the
    paging decision reads the ids on the host, so the steps cannot be
    graph-captured).  Device pager (device_tables): the slot tables on the
    device, misses copied from the pinned host mirror of the layer; the
    `steps` steps are one HIP graph, timed with HIP events."""
    import shutil
    import tempfile
    import time

    import torch

    from compressai_amd import paged, synth

    g = torch.Generator().manual_seed(7000)
    gui = torch.randint(-32768, 32768, (E, 1024, 256), generator=g, dtype=torch.int32).to(torch.int16)
    gus = (torch.rand(E, 1024, generator=g) + 0.5).to(torch.float16)
    dni = torch.randint(-32768, 32768, (E, 2048, 64), generator=g, dtype=torch.int32).to(torch.int16)
    dns = (torch.rand(E, 2048, generator=g) + 0.5).to(torch.float16)
    tmp = tempfile.mkdtemp(prefix="vq2m_")
    res = {}
    try:
        path = os.path.join(tmp, "layer.vq2m")
        paged.write_vq2m(path, [gui], [gus], [dni], [dns])
        store = paged.Vq2mStore(path)
        cb = synth.codebook(7001).to(dev)
        ids = torch.stack([torch.randperm(E, generator=g)[:8] for _ in range(steps)]).to(dev)
        w = torch.full((1, 8), 1.0 / 8, device=dev)
        h = synth.activations(7004, (1, 2048), dtype=torch.float16).to(dev)
        # device pager: sorted slot pool and one-launch sorted MoE (the
        # default), and the reference-layout slots on the gather kernels
        for name, cap, on_dev, srt in (("warm", E, False, None), ("churn", 16, False, None),
                                       ("warm_device", E, True, None), ("churn_device", 16, True, None),
                                       ("warm_device_gather_kernels", E, True, False)):
            layer = paged.PagedMoEExperts(0, store, cb, capacity=cap, device=dev, out_dtype=torch.float32,
                                          device_tables=on_dev, sorted_layout=srt)
            rec = layer.pager.mirror_record_bytes if layer.pager.sorted_layout else store.record_bytes
            for s_ in range(min(steps, 2 * E)):  # fill the pool / reach the steady state
                layer(h, ids[s_ % steps].view(1, 8), w)
            torch.cuda.synchronize(dev)
            m0 = layer.pager.misses
            if on_dev:
                gr = capture(lambda l: layer(h, ids[l].view(1, 8), w), steps, dev)
                m0 = layer.pager.misses
                time_graph(gr, 1, dev)
                dt = statistics.median(time_graph(gr, 1, dev)[0] for _ in range(REPEATS)) * 1e-3
                reps = 1 + REPEATS
                del gr
            else:
                t0 = time.perf_counter()
                for s_ in range(steps):
                    layer(h, ids[s_].view(1, 8), w)
                torch.cuda.synchronize(dev)
                dt = time.perf_counter() - t0
                reps = 1
            misses = (layer.pager.misses - m0) / reps
            res[name] = {"us_per_layer": round(dt * 1e6 / steps, 2), "misses_per_step": round(misses / steps, 2),
                         "feed_gbps": round(misses * rec / dt / 1e9, 2), "record_bytes": rec}
            log(f"paged MoE ({name}, {cap} slots of {E}): {res[name]['us_per_layer']:.1f} us/layer, "
                f"{res[name]['misses_per_step']:.2f} misses/step, {res[name]['feed_gbps']:.2f} GB/s fed")
            del layer
        store.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return res


# -------------------------------------------------------------- CPU baseline
def _cpu_info():
    import platform

    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _time_cpu(fn, budget_s):
    """Median of up to 20 timed runs after one warm-up, at least 3, bounded
    by about budget_s seconds of CPU work."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    runs = int(max(3, min(20, budget_s / max(first, 1e-3))))
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), runs


def cpu_baseline(dl, budget_s=20.0):
    """The reference CPU path (PackedLinear fallback, fp32) on the host for
    one configs[1] layer step, on all host cores."""
    import torch

    from oracle.ref_cpu_path import CpuRot, packed_linear_fallback

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    lay = {k: tuple(t.cpu() if hasattr(t, "cpu") else t for t in v[:5]) for k, v in dl.layers[0].items()}
    cb0, cb1 = dl.cb0.cpu(), dl.cb1.cpu()
    rot_h = CpuRot(dl.perm_h.cpu(), dl.sign_h.cpu(), 2048)
    rot_i = CpuRot(dl.perm_i.cpu(), dl.sign_i.cpu(), 2048)
    xa, xo, xm, xd = dl.x_attn.cpu(), dl.x_o.cpu(), dl.x_mlp.cpu(), dl.x_down.cpu()

    def step():
        for name, x, rot in (("q", xa, rot_h), ("k", xa, rot_h), ("v", xa, rot_h), ("o", xo, rot_h),
                             ("gate", xm, rot_h), ("up", xm, rot_h), ("down", xd, rot_i)):
            i0, i1, s, out, n = lay[name]
            packed_linear_fallback(x, rot, i0, i1, cb0, cb1 if i1 is not None else None, s)

    med, runs = _time_cpu(step, budget_s)
    cpu = _cpu_info()
    gbps = dl.bytes_per_step / med / 1e9
    log(f"cpu baseline: {med * 1e3:.1f} ms/step median of {runs} on {cores} threads ({cpu}) -> {gbps:.3f} GB/s")
    return {"value": round(gbps, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"configs[1] one layer step (q,k,v,o,gate,up,down + 4 RHTs), reference PackedLinear "
                      f"fp32 fallback restated in torch (oracle/ref_cpu_path.py); median of {runs} runs, "
                      f"{med * 1e3:.1f} ms/step; CPU: {cpu}"}


def cpu_moe_baseline(moe, budget_s=10.0):
    """The reference CPU path of the config-4 MoE layer on the host: router,
    then per token the vq_moe_parallel_gate_up_cpu / _down_cpu twins over the
    8 routed + 1 shared expert with fp32 codebooks (as the reference's CPU
    test feeds them), the two rotations, SwiGLU and the weighted combine
    (oracle/ref_cpu_path.moe_layer_cpu), for T = 1 and T = 8 on one layer of
    the benchmark's pool; all host cores."""
    import torch

    from oracle.ref_cpu_path import CpuRot, moe_layer_cpu

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    layer = moe["cpu_layer"]
    m = layer.experts_mod
    cb = m.cb16.float().cpu()
    gu, gus, dn, dns = (t.cpu() for t in (m.gate_up_idx, m.gate_up_scale, m.down_idx, m.down_scale))
    gate = layer.shared_gate.cpu()
    rot_h = CpuRot(m.rot_h.perm.cpu(), m.rot_h.sign.float().cpu(), m.rot_h.hb)
    rot_i = CpuRot(m.rot_i.perm.cpu(), m.rot_i.sign.float().cpu(), m.rot_i.hb)
    res = {}
    for T in (1, 8):
        h, lg = (t.cpu() for t in moe[T]["cpu_inputs"])
        med, runs = _time_cpu(lambda: moe_layer_cpu(h, lg, cb, gu, gus, dn, dns, gate, rot_h, rot_i,
                                                    top_k=layer.top_k, shared_id=layer.n_routed), budget_s)
        res[f"t{T}"] = {"us_per_layer": round(med * 1e6, 1), "runs": runs,
                        "gpu_speedup": round(med * 1e6 / moe[T]["us"], 1)}
        log(f"cpu moe baseline T={T}: {med * 1e3:.2f} ms/layer median of {runs} on {cores} threads")
    return {"unit": "us per MoE layer", "cores": cores, "kind": "port", "cpu": _cpu_info(),
            "sample": "configs[3] one MoE layer (router top-8 of 256 + shared expert, 2 bpw experts), "
                      "reference vq_moe_parallel_*_cpu composition restated in torch (oracle/ref_cpu_path.py), "
                      "fp32 codebook", **res}


def traffic_from_profiles():
    """HBM bytes per call of the dominant launch (the sorted gate+up kernel),
    from the committed rocprofv3 --pmc summary
    (profiles/sorted_gate_up_pmc.json), if present."""
    p = ROOT / "profiles" / "sorted_gate_up_pmc.json"
    try:
        return json.loads(p.read_text()).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--layers", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-lmhead", action="store_true")
    ap.add_argument("--no-small-m", action="store_true")
    ap.add_argument("--only", choices=["dominant", "dominant_gather", "dense", "copy", "moe", "paged", "lmhead",
                                       "small_m"], default=None)
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for {max(args.gpus, world)}); the VQ2 decode "
              "path would shard by output rows (dense) and by experts (MoE), which is designed, not built",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from compressai_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    log(f"device: {torch.cuda.get_device_name(0)}, {torch.cuda.get_device_properties(0).multi_processor_count} CUs")

    if args.only in ("dominant", "dominant_gather"):
        dl = DenseLayers(args.layers, dev)
        fn = dl.sorted if args.only == "dominant" else dl.fused
        for l in range(args.layers):
            fn(dl.layers[l], ("gate", "up"), dl.x_mlp, dl.perm_h, dl.sign_h)
        torch.cuda.synchronize(dev)
        log(f"{args.only}-only run done")
        return
    if args.only == "dense":
        dl = DenseLayers(args.layers, dev)
        for l in range(args.layers):
            dl.step(l)
        torch.cuda.synchronize(dev)
        log("dense-only run done")
        return
    if args.only == "small_m":
        bench_small_m(args, dev)
        log("small_m-only run done")
        return
    if args.only == "lmhead":
        bench_lm_head(args, dev, batch=1, copies=args.layers, only=True)
        log("lmhead-only run done")
        return
    if args.only == "paged":
        bench_paged(args, dev)
        return
    if args.only == "moe":
        res = bench_moe(args, dev, n_layers=args.layers)
        log("moe-only run done: " + ", ".join(f"T={T} {res[T]['us']:.2f} us" for T in (1, 8)))
        return
    if args.only == "copy":
        a = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize(dev)
        log("copy calibration: 4 x 64 MiB device copies done")
        return

    d = bench_dense(args, dev)
    moe = None if args.no_moe else bench_moe(args, dev)
    lm1 = None if args.no_lmhead else bench_lm_head(args, dev, batch=1)
    lm4 = None if args.no_lmhead else bench_lm_head(args, dev, batch=4)
    sm = None if args.no_small_m else bench_small_m(args, dev)
    up = None if args.no_small_m else bench_unpack(args, dev)
    pgd = None if args.no_moe else bench_paged(args, dev)
    cpu = None if args.no_cpu else cpu_baseline(d["dense"])
    cpu_moe = None if (args.no_cpu or moe is None) else cpu_moe_baseline(moe)
    c0 = bench_config0(args, dev)

    rec = {
        "metric": metric_name(),
        "value": round(d["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": d["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "configs[1]: dense decoder-layer projection set, batch 1, hidden 2048 (q,k,v,o 2 bpw; "
                        "gate,up,down 4 bpw; RHT 2048 x3 + 6144, each with permutation + signs); fp16 codebooks/"
                        "scales/activations, fp32 out; q/k/v in one code-sorted launch (PackedProjections), o, "
                        "gate/up, down on the code-sorted layout (PackedLinear), batch 1",
            "layers_cycled": min(d["layers"], d["steps"]),
            "layer_sets_resident": d["layers"],
            "bytes_per_step": d["bytes_per_step"],
            "graph_replay": True,
        },
        "pct_of_peak": round(100.0 * d["gbps"] / PEAK_HBM_GBPS, 3),
        "resident_index_bytes": {
            "note": "index bytes held on the device per unit: the reference planes (2 bytes per code, the public "
                    "format) and the code-sorted copies the batch-1 kernels read (~3.06 bytes per code; the MoE "
                    "layer's down pool twice, in 9 chunks for T = 1 and 5 taller ones for T >= 2); both are "
                    "resident unless the owner releases the planes",
            "dense_layer": {"planes": d["plane_bytes"], "sorted": d["sorted_bytes"]},
            "moe_layer_257_experts": None if moe is None else moe["resident"],
            "lm_head": None if lm1 is None else {"planes": lm1["plane_bytes"], "sorted": lm1["sorted_bytes"]},
        },
        "moe_layer_us": None if moe is None else round(moe[1]["us"], 3),
        "moe_layer_gbps": None if moe is None else round(moe[1]["gbps"], 2),
        "moe_layer_us_t8": None if moe is None else round(moe[8]["us"], 3),
        "moe_layer_gbps_t8": None if moe is None else round(moe[8]["gbps"], 2),
        "lm_head_us_b1": None if lm1 is None else round(lm1["us"], 3),
        "lm_head_gbps_b1": None if lm1 is None else round(lm1["gbps"], 2),
        "lm_head_us_b4": None if lm4 is None else round(lm4["us"], 3),
        "lm_head_gbps_b4": None if lm4 is None else round(lm4["gbps"], 2),
        "lm_head_us_b4_matrix_cores": None if lm4 is None else round(lm4["matrix_cores_us"], 3),
        "lm_head_us_b1_prerotated": None if lm1 is None else round(lm1["prerotated_us"], 3),
        "lm_head_us_b1_gather_kernel": None if lm1 is None else round(lm1["gather_us"], 3),
        "dense_step_us_gather_kernel": round(d["gather_step_us"], 3),
        "gate_up_us_gather_kernel": round(d["dom_gather_us"], 3),
        "config0": c0,
        "dense_spread_us": d["spread_us"],
        "timing": f"median of {REPEATS} timed repetitions of the steps (HIP events on the replay stream)",
        "small_m": sm,
        "unpack_fixed": up,
        "paged_moe_t1": pgd,
        "roofline": {
            "kernel": "vq_sorted_kernel<1,3,1,0> (RHT 2048 in the prologue, slice sum in the launch), "
                      "gate+up: 2 x 4 bpw (16,16) 6144 x 2048, batch 1, one call = one launch",
            "bound": "hbm",
            "achieved": round(d["dom_gbps"], 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(d["dom_gbps"] / PEAK_HBM_GBPS, 5),
            "traffic": traffic_from_profiles(),
            "traffic_source": "profiles/sorted_gate_up_pmc.json: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of "
                              "bench.py --only dominant --layers 8, scaled by a 64 MiB copy (stored profile, "
                              "not this run)",
            "us_per_launch": round(d["dom_us"], 3),
            "algorithmic_bytes_per_launch": d["dom_bytes"],
        },
        "cpu_baseline": cpu,
        "cpu_baseline_moe": cpu_moe,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
