"""Dense packed-linear callers of the VQ GEMV (reference: vq2/runtime.py).

``PackedLinear(shape, cfg, tag, idx, scale, cbs, device)`` keeps the
reference constructor (vq2/runtime.py:70-80): ``idx`` is the list of index
planes (int16 for 16-bit stages, uint8 for 8-bit stages), ``scale`` the
per-row scales, ``cbs`` a dict of codebooks keyed by the cfg prefix
("16", "16_8", "16_16").  ``forward(x)`` rotates x with the layer's RHT and
runs the fused VQ GEMV (batch <= 2) or the matrix-core small-M GEMM
(batch >= 3) for every cfg in (16,), (16, 8), (16, 16) -- the reference
fuses only batch 1 of (16,) and (16, 8) and otherwise re-materialises the
dequantized matrix (runtime.py:91-110).
``PackedLMHead`` (runtime.py:136-144) wraps it and adds ``argmax``.
``PackedProjections`` runs projections of one activation (q, k, v) in one
launch.

Large matrices (``SORTED_MIN_CODES`` codes or more, 2 and 4 bpw) also keep
a code-sorted copy of their index planes (``kernels.SortedPlanes``, packed
once here): at batch 1 their GEMV and the LM head's top-1 run on it, sorted
gathers sharing codebook lines.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import kernels as K
from .rot import get_rot


def cfg_key(cfg, i):
    return "_".join(str(b) for b in cfg[: i + 1])


# batch rows per matrix-core launch (vq2_gemm_small_m takes up to 64)
SMALL_M_MAX = 64

# matrices with at least this many codes (all stages) use the code-sorted
# layout at batch 1.  Measured on MI355X: gate + up (2 x 6144 x 2048, 4 bpw)
# 15.0 us against 29.6 us, down (2048 x 6144, 4 bpw) 12.3 against 20.1, the
# 151936 x 2048 LM head 55 against 171; the 2048 x 2048 o projection
# (0.5 M codes) 7.1 against 8.5 us, with the small-matrix chunking (about
# 0.75 x CUs chunks of 11 rows, one workgroup each; 9.0 us at 9 chunks of
# 228 rows x 8 slices).
SORTED_MIN_CODES = 1 << 19
# a launch of several projections of one activation (PackedProjections) uses
# the code-sorted layout at batch 1 from this many codes on, its members
# repacked to one chunk height over the launch's rows (about 0.75 x CUs
# chunks).  Measured on MI355X: q, k and v of the 2048-wide attention
# (0.79 M codes, 192 chunks of 16 rows) 7.6 us against 11.4 us on the gather
# kernel; o alone (0.52 M codes, above) 7.1 against 8.5.
SORTED_MIN_LAUNCH_CODES = SORTED_MIN_CODES
# Batch 2-4 on the sorted layout (vq_sorted_gemm_batch: one centroid gather
# for every activation row, the activation rotated by its own launch first)
# where it was measured faster (HIP graphs, MI355X, us per call):
#  * matrices of SORTED_BATCH_MIN_CODES codes or more -- the LM head
#    151936 x 2048: 68.5 against 195.6 (gather kernel) at batch 2, 122
#    (2-row workgroups over both row pairs) against 181 (matrix cores) at
#    batch 4, top-1 or logits;
#  * batch 2 of inputs wider than 2048 (down 2048 x 6144, 4 bpw: 22.4 against
#    28.9 on the gather kernel with the 6144-point RHT in its prologue);
#  * PackedProjections at batch 3-4 (q, k, v in one launch: 22.0-24.4 against
#    35.9-36.1 for the three projections on the matrix cores; gate + up:
#    40.1-42.0 against 47.0-47.4), and at batch 2 with
#    SORTED_BATCH2_LAUNCH_MIN_CODES codes or more (gate + up: 24.6 against
#    37.6 in one gather-kernel launch).
# Not used where it was slower: one 6144 x 2048 4 bpw matrix at batch 2
# (23.2 against 20.9) and 3-4 (32-35 against 24 on the matrix cores), the
# down matrix at batch 3-4 (35-39 against 25), q / k / v at batch 2 (17.6
# against 12.9; 0.79 M codes).
SORTED_BATCH = True
SORTED_BATCH_MIN_CODES = 8 << 20
# PackedProjections at batch 2 on the sorted layout from this many codes on
# (gate + up, 6.3 M codes: faster; q, k, v, 0.79 M codes: slower)
SORTED_BATCH2_LAUNCH_MIN_CODES = 2 << 20
# the sorted kernel builds the RHT in LDS up to this width, else x is rotated first
SORTED_FUSED_RHT_MAX_N = 8192


def vq_matmul(xr, i0, i1, cb0, cb1, scale, out, n, out_dtype, y=None):
    """y [B, out] = VQ(W) . xr for rotated xr [B, n], B >= 1: the batched
    GEMV below 3 rows, the matrix-core GEMM (every centroid gathered once per
    64 rows) from 3 rows on."""
    B = xr.shape[0]
    if B < 3 or n % 64:
        return K.vq_gemv(xr, i0, i1, cb0, cb1, scale, out, n, 1.0, out_dtype=out_dtype, y=y)
    if y is None:
        y = torch.empty((B, out), dtype=out_dtype, device=xr.device)
    for b0 in range(0, B, SMALL_M_MAX):
        b1 = min(B, b0 + SMALL_M_MAX)
        K.vq_gemm_small_m(xr[b0:b1], i0, i1, cb0, cb1, scale, out, n, 1.0, y=y[b0:b1])
    return y


class PackedLinear(nn.Module):
    """``scale_dtype``: the row scales are held in bf16 by default, as the
    reference rounds them at construction (vq2/runtime.py:78); ``None`` keeps
    the given dtype (e.g. the container's fp16 scales, one rounding fewer)."""

    def __init__(self, shape, cfg, tag, idx, scale, cbs, device, act_dtype=torch.float32,
                 scale_dtype=torch.bfloat16, sorted_layout=None):
        super().__init__()
        self.out, self.n = int(shape[0]), int(shape[1])
        self.cfg, self.tag = tuple(cfg), tag
        if self.cfg not in ((16,), (16, 8), (16, 16)):
            raise K.Vq2Error(f"unsupported cfg {self.cfg}")
        self.keys = [cfg_key(self.cfg, i) for i in range(len(self.cfg))]
        for i, a in enumerate(idx):
            self.register_buffer(f"idx{i}", a.to(device).contiguous(), persistent=False)
        self.register_buffer("scale", scale.to(device=device, dtype=scale_dtype or scale.dtype).contiguous(),
                             persistent=False)
        self._cbs = [cbs]
        self.rot = get_rot(tag, self.n, device)
        self.act_dtype = act_dtype
        # code-sorted copy of the planes for the batch-1 GEMV of large matrices
        codes = self.out * (self.n // 8) * len(self.cfg)
        dev = torch.device(device)
        use = sorted_layout if sorted_layout is not None else (
            codes >= SORTED_MIN_CODES and dev.type == "cuda" and self.cfg in ((16,), (16, 8), (16, 16)))
        self.sorted = None
        if use:
            self.sorted = K.SortedPlanes(self.idx0, getattr(self, "idx1", None), self.out, self.n, device=dev)

    def _planes(self):
        i1 = getattr(self, "idx1", None)
        cb0 = self._cbs[0][self.keys[0]]
        cb1 = self._cbs[0][self.keys[1]] if len(self.keys) > 1 else None
        return self.idx0, i1, cb0, cb1

    @property
    def planes_released(self):
        return self.idx0 is None

    def release_planes(self):
        """Frees the reference index planes and keeps only the code-sorted
        copy (~3.06 bytes per code resident instead of ~5.06 with both):
        batch 1 runs on it as before, every other batch on the sorted batch
        kernel in launches of up to 4 rows after the RHT (the activation held
        in fp16 under a power-of-two scale per row, ~1e-4 of max |y|).  Needs
        the sorted copy, fp16 / bf16 codebooks and a chunk height the batch
        kernel fits; the planes cannot be restored.  A PackedProjections over
        this module must be built before (it may repack the planes)."""
        if self.planes_released:
            return
        cb0 = self._cbs[0][self.keys[0]]
        if self.sorted is None:
            raise K.Vq2Error("release_planes: no code-sorted copy to run on")
        if cb0.dtype not in (torch.float16, torch.bfloat16):
            raise K.Vq2Error("release_planes: the sorted kernels take fp16 / bf16 codebooks")
        if not (K.sorted_batch_fits([self.sorted], 4) and K.sorted_batch_fits([self.sorted], 2)):
            raise K.Vq2Error("release_planes: the sorted batch kernel does not fit these chunks")
        for i in range(len(self.cfg)):
            setattr(self, f"idx{i}", None)

    def _sorted_rows(self, x2, od):
        """Batch >= 2 without the planes: the sorted batch kernel over groups
        of up to 4 rotated rows."""
        _, _, cb0, cb1 = self._planes()
        xr = self.rot.fwd(x2, out_dtype=torch.float32)
        y = torch.empty((x2.shape[0], self.out), dtype=od, device=x2.device)
        for b0 in range(0, x2.shape[0], K.SORTED_BATCH_MAX):
            b1 = min(x2.shape[0], b0 + K.SORTED_BATCH_MAX)
            K.vq_sorted_gemm_batch(xr[b0:b1], [(self.sorted, self.scale)], cb0, cb1, self.n, out_dtype=od,
                                   ys=[y[b0:b1]])
        return y

    def _sorted_ok(self, B, cb0):
        return self.sorted is not None and B == 1 and cb0.dtype in (torch.float16, torch.bfloat16)

    def _sorted_batch_ok(self, B, cb0):
        """Batch 2-4 on the sorted layout, where it was measured faster (see
        SORTED_BATCH)."""
        if not (SORTED_BATCH and self.sorted is not None and 2 <= B <= K.SORTED_BATCH_MAX
                and cb0.dtype in (torch.float16, torch.bfloat16) and K.sorted_batch_fits([self.sorted], B)):
            return False
        codes = self.out * (self.n // 8) * len(self.cfg)
        return codes >= SORTED_BATCH_MIN_CODES or (B == 2 and self.n > 2048)

    def _sorted_args(self, x1):
        """(x, perm, sign, hb, rht scale) for a sorted launch: the RHT built in
        the kernel up to SORTED_FUSED_RHT_MAX_N, else x rotated first."""
        r = self.rot
        if self.n % 64 == 0 and self.n <= SORTED_FUSED_RHT_MAX_N:
            return x1, r._perm32, r._sign8, r.hb, r.scale
        return r.fwd(x1, out_dtype=torch.float32), None, None, 0, 1.0

    def forward(self, x, out_dtype=None):
        x2 = x.reshape(-1, self.n).contiguous()
        i0, i1, cb0, cb1 = self._planes()
        od = out_dtype or x.dtype
        B = x2.shape[0]
        if self._sorted_ok(B, cb0):
            xs, perm, sign, hb, sc = self._sorted_args(x2.reshape(-1))
            y = K.vq_sorted_gemv(xs, [(self.sorted, self.scale)], cb0, cb1, self.n, perm, sign, hb, sc,
                                 out_dtype=od)[0]
        elif self._sorted_batch_ok(B, cb0):
            xr = self.rot.fwd(x2, out_dtype=torch.float32)
            y = K.vq_sorted_gemm_batch(xr, [(self.sorted, self.scale)], cb0, cb1, self.n, out_dtype=od)[0]
        elif self.planes_released:
            y = self._sorted_rows(x2, od)
        elif B <= 2 and self.n % 64 == 0:
            # one launch: every workgroup rotates x in LDS, then multiplies
            y = K.vq_gemv_rht(x2, [(i0, i1, self.scale, self.out)], cb0, cb1, self.n, self.rot._perm32,
                              self.rot._sign8, self.rot.hb, self.rot.scale, out_dtype=od)[0]
        else:
            xr = self.rot.fwd(x2, out_dtype=self.act_dtype)
            y = vq_matmul(xr, i0, i1, cb0, cb1, self.scale, self.out, self.n, od)
        return y.view(*x.shape[:-1], self.out)

    def nbytes(self):
        own = sum(b.numel() * b.element_size() for b in self.buffers())
        return own + (self.sorted.nbytes() if self.sorted is not None else 0)


class PackedProjections(nn.Module):
    """Projections of one activation in one launch: ``PackedLinear``s of the
    same width, cfg, codebooks and rotation tag, e.g. q, k and v of an
    attention layer (the reference's quantizer gives them all the tag
    "attn", vq2/quantize_35b.py:146-161, so they share the RHT of the input).
    ``forward(x)`` returns the list of the projections' outputs, each what the
    projection's own forward gives (vq2/runtime.py:91-110, once per matrix
    there): with the sorted layout (the matrices hold
    ``SORTED_MIN_LAUNCH_CODES`` codes or more together) one sorted launch at
    batch 1 and one sorted batch launch after the RHT at batch 3-4, and at
    batch 2 with ``SORTED_BATCH2_LAUNCH_MIN_CODES`` codes or more (gate +
    up); else one
    gather-kernel launch with the RHT built in for batch <= 2; other batches
    run each projection.  Up to 4 projections."""

    def __init__(self, linears, sorted_layout=None):
        super().__init__()
        lins = list(linears)
        if not 1 <= len(lins) <= 4:
            raise K.Vq2Error("PackedProjections: 1..4 projections")
        a = lins[0]
        for m in lins[1:]:
            if m.n != a.n or m.cfg != a.cfg or m.tag != a.tag or m._cbs[0] is not a._cbs[0]:
                raise K.Vq2Error("PackedProjections: the projections must share width, cfg, codebooks and tag")
            if m.scale.dtype != a.scale.dtype:
                raise K.Vq2Error("PackedProjections: the projections must share the scale dtype")
        self.lins = nn.ModuleList(lins)
        codes = sum(m.out * (m.n // 8) * len(m.cfg) for m in lins)
        self.codes = codes
        dev = a.scale.device
        use = sorted_layout if sorted_layout is not None else (
            codes >= SORTED_MIN_LAUNCH_CODES and dev.type == "cuda" and a.cfg in ((16,), (16, 8), (16, 16)))
        self.sorted = None
        if use:
            # a launch of fewer than 2^20 codes (q, k, v): one chunk height
            # over the launch's rows (about 0.75 x CUs chunks); the members
            # then hold these planes (one sorted copy per matrix)
            R = K.sorted_launch_rows_per_chunk([m.out for m in lins], a.n // 8, dev) if dev.type == "cuda" else None
            self.sorted = []
            for m in lins:
                sp = m.sorted
                if sp is None or (R is not None and sp.rows_per_chunk != R):
                    if m.planes_released:
                        raise K.Vq2Error("PackedProjections: a projection's planes were released before its "
                                         "sorted copy could be packed for this launch")
                    sp = K.SortedPlanes(m.idx0, getattr(m, "idx1", None), m.out, m.n, device=dev, rows_per_chunk=R)
                    m.sorted = sp
                self.sorted.append(sp)

    def forward(self, x, out_dtype=None):
        lins = self.lins
        a = lins[0]
        x2 = x.reshape(-1, a.n).contiguous()
        i0, i1, cb0, cb1 = a._planes()
        od = out_dtype or x.dtype
        B = x2.shape[0]
        if self.sorted is not None and B == 1 and cb0.dtype in (torch.float16, torch.bfloat16):
            xs, perm, sign, hb, sc = a._sorted_args(x2.reshape(-1))
            ys = K.vq_sorted_gemv(xs, [(sp, m.scale) for sp, m in zip(self.sorted, lins)], cb0, cb1, a.n, perm,
                                  sign, hb, sc, out_dtype=od)
        elif (SORTED_BATCH and self.sorted is not None and 2 <= B <= K.SORTED_BATCH_MAX
              and (B >= 3 or self.codes >= SORTED_BATCH2_LAUNCH_MIN_CODES)
              and cb0.dtype in (torch.float16, torch.bfloat16) and K.sorted_batch_fits(self.sorted, B)):
            xr = a.rot.fwd(x2, out_dtype=torch.float32)
            ys = K.vq_sorted_gemm_batch(xr, [(sp, m.scale) for sp, m in zip(self.sorted, lins)], cb0, cb1, a.n,
                                        out_dtype=od)
        elif any(m.planes_released for m in lins):
            return [m(x, out_dtype=out_dtype) for m in lins]
        elif B <= 2 and a.n % 64 == 0:
            mats = []
            for m in lins:
                mi0, mi1, _, _ = m._planes()
                mats.append((mi0, mi1, m.scale, m.out))
            ys = K.vq_gemv_rht(x2, mats, cb0, cb1, a.n, a.rot._perm32, a.rot._sign8, a.rot.hb, a.rot.scale,
                               out_dtype=od)
        else:
            return [m(x, out_dtype=out_dtype) for m in lins]
        return [y.view(*x.shape[:-1], m.out) for y, m in zip(ys, lins)]


class PackedLMHead(nn.Module):
    """lm_head sharing the packed weights of a PackedLinear."""

    def __init__(self, lin: PackedLinear):
        super().__init__()
        self.lin = lin

    def forward(self, x):
        return self.lin(x)

    def argmax(self, x):
        """Top-1 token per row of x without materialising bf16 logits:
        (idx int64 [B], logit fp32 [B])."""
        lin = self.lin
        x2 = x.reshape(-1, lin.n).contiguous()
        i0, i1, cb0, cb1 = lin._planes()
        if lin._sorted_ok(x2.shape[0], cb0):
            xs, perm, sign, hb, sc = lin._sorted_args(x2.reshape(-1))
            return K.vq_sorted_gemv_argmax(xs, lin.sorted, lin.scale, cb0, cb1, lin.n, perm, sign, hb, sc)
        if lin._sorted_batch_ok(x2.shape[0], cb0):
            xr = lin.rot.fwd(x2, out_dtype=torch.float32)
            return K.vq_sorted_gemm_batch_argmax(xr, lin.sorted, lin.scale, cb0, cb1, lin.n)
        if lin.planes_released:
            xr = lin.rot.fwd(x2, out_dtype=torch.float32)
            parts = [K.vq_sorted_gemm_batch_argmax(xr[b0:b0 + K.SORTED_BATCH_MAX], lin.sorted, lin.scale, cb0, cb1,
                                                   lin.n) for b0 in range(0, x2.shape[0], K.SORTED_BATCH_MAX)]
            return torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])
        xr = lin.rot.fwd(x2, out_dtype=lin.act_dtype)
        return K.vq_gemv_argmax(xr, i0, i1, cb0, cb1, lin.scale, lin.out, lin.n, 1.0)
