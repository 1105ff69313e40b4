"""Drop-in VQ entry points of ``vq2.kernels`` backed by hand-written HIP
kernels for gfx950 (libvq2_amd.so, C ABI in include/vq2_amd.h).

Kept names and signatures (reference: vq2/kernels.py):
  vq_gemv_16(xr, i0, cb0, scale, out, n, rs=1.0) -> y[out] bf16        (224-230)
  vq_gemv_16_8(xr, i0, i1, cb0, cb1, scale, out, n, rs=1.0) -> y bf16  (215-221)
  vq_moe_parallel_gate_up(xr, topk_ids, gate_up_idx, cb16, gate_up_scale,
                          y_out, OUT=1024, NG=256, rs=1.0) -> None      (246-254)
  vq_moe_parallel_down(act_r, topk_ids, down_idx, cb16, down_scale,
                       y_out, OUT=2048, NG=64, rs=1.0) -> None           (256-264)
  HAVE_TRITON, FUSED_KERNELS_ENABLED, set_fused_kernels_enabled           (9-20)
  patch_transformers_kernels, optimize_deltanet_layers (no-ops here: the
  attention / DeltaNet fusions they install are outside this library)

Additive entry points: vq_gemv_16_16 (4 bpw), batched GEMV (x of shape
[B, n]), vq_rht, vq_swiglu_rht, vq_router_topk, vq_moe_down_combine,
vq_gemv_argmax, vq_argmax, vq_dequant_rows, vq_decode_idx.

Every entry launches on the current torch stream of the input's device and
raises ``Vq2Error`` (a RuntimeError) on any invalid argument.  There is no CPU
or Triton fallback: CPU tensors are rejected and a missing library raises
ImportError.  Differences from the reference kernels: any OUT (no silent
tail drop from ``OUT // BR``), ids may be int32 or int64, an id outside the
pool yields NaN rows instead of an out-of-bounds read, and the output dtype
is selectable (``out_dtype``; bf16 by default, as in the reference).
"""
from __future__ import annotations

import ctypes
import weakref

import torch

from . import _lib
from ._lib import Vq2Error

__all__ = [
    "HAVE_TRITON", "FUSED_KERNELS_ENABLED", "set_fused_kernels_enabled",
    "vq_gemv_16", "vq_gemv_16_8", "vq_gemv_16_16", "vq_gemv",
    "vq_moe_parallel_gate_up", "vq_moe_parallel_down", "vq_moe_down_combine", "vq_moe_grouped",
    "vq_gemv_rht", "vq_moe_gate_up_rht", "vq_moe_down_swiglu_combine", "vq_gemm_small_m",
    "vq_moe_router_gate_up_rht", "vq_unpack_fixed", "SortedPlanes", "vq_sorted_gemv", "vq_sorted_gemv_argmax",
    "vq_rht", "vq_swiglu_rht", "vq_router_topk", "vq_gemv_argmax", "vq_argmax",
    "vq_dequant_rows", "vq_decode_idx", "patch_transformers_kernels",
    "optimize_deltanet_layers", "Vq2Error",
]


def _library_available() -> bool:
    try:
        _lib.load()
        return True
    except (ImportError, OSError):
        return False


# "fused GPU kernels available" (the reference's meaning of HAVE_TRITON)
HAVE_TRITON = _library_available() and torch.cuda.is_available()

FUSED_KERNELS_ENABLED = True


def set_fused_kernels_enabled(enabled: bool):
    """Reference A/B switch (vq2/kernels.py:16-20).  Kept for callers; the VQ
    entry points below always run the HIP kernels."""
    global FUSED_KERNELS_ENABLED
    FUSED_KERNELS_ENABLED = bool(enabled)


def patch_transformers_kernels():
    """Out of scope here (the reference installs attention/DeltaNet Triton
    fusions, vq2/kernels.py:572-726).  No-op; returns False."""
    return False


def optimize_deltanet_layers(model):
    """Out of scope here (vq2/kernels.py:443-565).  Returns model unchanged."""
    return model


# ------------------------------------------------------------------ helpers
_DT = {torch.float32: _lib.DT_F32, torch.float16: _lib.DT_F16, torch.bfloat16: _lib.DT_BF16}


def _dt(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise Vq2Error(f"{what}: unsupported dtype {t.dtype} (float32/float16/bfloat16)") from None


def _dev(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise Vq2Error("libvq2_amd kernels need GPU tensors (no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise Vq2Error(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _contig(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_contiguous():
        raise Vq2Error(f"{what} must be contiguous")
    return t


def _stream(dev: torch.device):
    return torch.cuda.current_stream(dev).cuda_stream


def _p(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _idx16(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dtype == torch.uint16:
        t = t.view(torch.int16)
    if t.dtype != torch.int16:
        raise Vq2Error(f"{what}: index plane must be int16 (uint16 codes), got {t.dtype}")
    return _contig(t, what)


def _perm_sign(perm, sign, n, what="") -> None:
    """The kernels read n entries of each rotation table: perm int32 [n],
    sign int8 [n], contiguous (either may be None)."""
    for t, nm, dt in ((perm, "perm", torch.int32), (sign, "sign", torch.int8)):
        if t is not None and (t.dtype != dt or t.numel() != n or not t.is_contiguous()):
            raise Vq2Error(f"{what}{nm} must be a contiguous {dt} [{n}]")


def _gate_vec(gate, n, what="shared_gate") -> torch.Tensor:
    """A shared-expert gate vector: n contiguous fp32 / fp16 / bf16 values."""
    _contig(gate, what)
    if gate.numel() != n:
        raise Vq2Error(f"{what} must hold {n} values, got {gate.numel()}")
    _dt(gate, what)
    return gate


def _ids(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    if t.dtype == torch.int32:
        return _contig(t, "topk_ids"), _lib.ID_I32
    if t.dtype == torch.int64:
        return _contig(t, "topk_ids"), _lib.ID_I64
    raise Vq2Error(f"topk_ids must be int32 or int64, got {t.dtype}")


# --------------------------------------------------------------- dense GEMV
def _planes(i0, i1, cb0, cb1, scale, out, n):
    """Validate one matrix's index planes, codebooks and scales; returns
    (i0, i1, s2_kind) with the planes viewed as the kernels read them.
    Checks only shapes, dtypes and layout (no device access), so the kernels
    never index past a plane, a codebook or the scales."""
    if n % 8:
        raise Vq2Error(f"n={n} must be a multiple of 8")
    i0 = _idx16(i0, "i0")
    if i0.numel() != out * (n // 8):
        raise Vq2Error(f"i0 has {i0.numel()} codes, expected out*n/8 = {out * (n // 8)}")
    s2 = _lib.S2_NONE
    if i1 is not None:
        if cb1 is None:
            raise Vq2Error("a stage-2 plane needs its codebook cb1")
        if cb1.dim() != 2 or cb1.shape[-1] != 8:
            raise Vq2Error(f"cb1 must be [K, 8], got {tuple(cb1.shape)}")
        if i1.dtype == torch.uint8:
            s2 = _lib.S2_U8
            if cb1.shape[0] < 256:
                raise Vq2Error("cb1 must have 256 rows for a uint8 stage-2 plane")
        else:
            i1 = _idx16(i1, "i1")
            s2 = _lib.S2_U16
            if cb1.shape[0] < 65536:
                raise Vq2Error("cb1 must have 65536 rows for an int16 stage-2 plane")
        _contig(i1, "i1")
        if i1.numel() != i0.numel():
            raise Vq2Error("i1 and i0 must have the same number of codes")
        _contig(cb1, "cb1")
        if cb1.dtype != cb0.dtype:
            raise Vq2Error("cb0 and cb1 must share a dtype")
    _contig(cb0, "cb0")
    if cb0.dim() != 2 or cb0.shape[-1] != 8 or cb0.shape[0] < 65536:
        raise Vq2Error(f"cb0 must be [65536, 8], got {tuple(cb0.shape)}")
    _dt(cb0, "cb0")
    _contig(scale, "scale")
    _dt(scale, "scale")
    if scale.numel() != out:
        raise Vq2Error(f"scale has {scale.numel()} entries, expected {out}")
    return i0, i1, s2


def check_gemv_rht_mats(mats, cb0, cb1, n):
    """Validate the matrices of one vq_gemv_rht launch: every matrix passes
    the single-matrix checks (planes, codebooks, scales) and all of them
    share the stage-2 kind and the scale dtype, which the launch passes once
    for every segment.  Returns (s2_kind, [(i0, i1, scale, out_rows)])."""
    if not 1 <= len(mats) <= 4:
        raise Vq2Error("vq_gemv_rht: 1..4 matrices per launch")
    s2 = sdt = None
    checked = []
    for k, (i0, i1, scale, out_rows) in enumerate(mats):
        out_rows = int(out_rows)
        i0v, i1v, s2k = _planes(i0, i1, cb0, cb1, scale, out_rows, n)
        if s2 is None:
            s2, sdt = s2k, scale.dtype
        elif s2k != s2:
            raise Vq2Error(f"vq_gemv_rht: matrix {k} has another stage-2 kind than matrix 0 "
                           "(all matrices of a launch share one cfg)")
        elif scale.dtype != sdt:
            raise Vq2Error(f"vq_gemv_rht: matrix {k} has {scale.dtype} scales, matrix 0 {sdt} "
                           "(the scales of a launch share a dtype)")
        checked.append((i0v, i1v, scale, out_rows))
    return s2, checked


def vq_gemv(xr, i0, i1, cb0, cb1, scale, out, n, rs=1.0, *, out_dtype=torch.bfloat16, y=None):
    """Generic VQ GEMV: 2 bpw (i1 None), 3 bpw (i1 uint8) or 4 bpw (i1 int16).
    xr [n] -> y [out]; xr [B, n] -> y [B, out]."""
    dev = _dev(xr, i0, i1, cb0, cb1, scale, y)
    n = int(n)
    out = int(out)
    x2 = xr.reshape(-1, n) if xr.dim() != 2 else xr
    if x2.shape[-1] != n or x2.stride(-1) != 1:
        raise Vq2Error(f"xr must have a unit-stride last dim of size n={n}")
    B = x2.shape[0]
    i0, i1, s2 = _planes(i0, i1, cb0, cb1, scale, out, n)
    if y is None:
        y = torch.empty((B, out) if xr.dim() == 2 else (out,), dtype=out_dtype, device=dev)
    else:
        _contig(y, "y")
        if y.numel() != B * out:
            raise Vq2Error("y has the wrong size")
    _lib.call("vq2_gemv", _p(x2), _dt(x2, "xr"), B, x2.stride(0) if B > 1 else n,
              _p(i0), _p(i1), s2, _p(cb0), _p(cb1), _dt(cb0, "cb0"), _p(scale), _dt(scale, "scale"),
              _p(y), _dt(y, "y"), out, out, n, float(rs), _stream(dev))
    return y


# Split-K partials of vq_gemm_small_m and the sorted launches (in a zeroed
# buffer of their own, the arrival counters and partials of vq_sorted_gemv),
# one buffer per
# (device, stream): launches on one stream run in order, so they can share
# it.  The buffers
# only grow, and a buffer that a larger one replaces is kept alive until the
# process ends: a HIP graph captured earlier holds its raw address and writes
# into it on every replay.
_WS: dict = {}
_WS_RETIRED: list = []


def _workspace(dev: torch.device, nbytes: int, *, sorted_kind: bool = False) -> torch.Tensor | None:
    """The workspace of this (device, stream).  vq_sorted_gemv and
    vq_sorted_moe share one of their own, allocated zeroed: it begins with
    arrival counters that must be zero before a launch (each call leaves them
    zero), which another kernel's partials must never overwrite."""
    if nbytes == 0:
        return None
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream, sorted_kind)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        alloc = torch.zeros if sorted_kind else torch.empty
        new = alloc(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        if buf is not None:
            if sorted_kind:  # the MoE status word carries over
                new[WS_STATUS:WS_STATUS + 4].copy_(buf[WS_STATUS:WS_STATUS + 4])
            _WS_RETIRED.append(buf)
        buf = new
        _WS[key] = buf
    return buf


# The sorted workspace's header (include/vq2_amd.h): arrival counters, and in
# its last 128-byte line the one-launch MoE's status word.
WS_HEADER = 16384
WS_STATUS = WS_HEADER - 128
MOE_WAIT_ID = 1      # a down workgroup gave up waiting for its pair's routed id
MOE_WAIT_COUNT = 2   # a down workgroup gave up waiting for its pair's gate_up sums


def vq_sorted_moe_status(device=None, *, clear=False) -> int:
    """Wait-timeout bits (MOE_WAIT_ID | MOE_WAIT_COUNT) that the one-launch
    MoE kernels left in this (device, stream)'s sorted workspace, read after
    the stream's queued work (a host synchronisation, so never inside graph
    capture).  0: no wait gave up.  A set bit means some pair's output was
    NaN because its wait gave up; clear=True resets the word."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    buf = _WS.get((dev.index, torch.cuda.current_stream(dev).cuda_stream, True))
    if buf is None:
        return 0
    st = int(_lib.load().vq2_sorted_moe_status(buf.data_ptr(), 1 if clear else 0, _stream(dev)))
    if st < 0:
        _lib.check(st, "vq2_sorted_moe_status")
    return st


def vq_sorted_moe_set_wait(max_polls=1 << 20, extra_arrivals=0) -> None:
    """Bound of each wait of the one-launch MoE (polls of >= 640 clocks) and
    an offset added to the gate_up count its down workgroups wait for, for
    all later launches of the process.  The defaults (2^20, 0) are the
    production values; tests of the give-up path pass a short bound and an
    unreachable count."""
    _lib.call("vq2_sorted_moe_set_wait", int(max_polls), int(extra_arrivals))


def vq_gemm_small_m(xr, i0, i1, cb0, cb1, scale, out, n, rs=1.0, *, out_dtype=torch.bfloat16, y=None):
    """Small-M batched VQ GEMM on the matrix cores: xr [B, n] (B <= 64,
    rotated) -> y [B, out], for 2 bpw (i1 None), 3 bpw (i1 uint8) or 4 bpw
    (i1 int16).  Replaces the batch > 1 fallback of PackedLinear
    (vq2/runtime.py:105-110): every centroid is gathered once for all B rows."""
    dev = _dev(xr, i0, i1, cb0, cb1, scale, y)
    n = int(n)
    out = int(out)
    x2 = xr.reshape(-1, n) if xr.dim() != 2 else xr
    if x2.shape[-1] != n or x2.stride(-1) != 1:
        raise Vq2Error(f"xr must have a unit-stride last dim of size n={n}")
    B = x2.shape[0]
    if not 1 <= B <= 64:
        raise Vq2Error(f"vq_gemm_small_m: batch {B} outside 1..64")
    i0, i1, s2 = _planes(i0, i1, cb0, cb1, scale, out, n)
    if y is None:
        y = torch.empty((B, out), dtype=out_dtype, device=dev)
    else:
        _contig(y, "y")
        if y.numel() != B * out:
            raise Vq2Error("y has the wrong size")
    lib = _lib.load()
    ws = _workspace(dev, int(lib.vq2_gemm_small_m_workspace(B, out, n)))
    _lib.call("vq2_gemm_small_m", _p(x2), _dt(x2, "xr"), B, x2.stride(0) if B > 1 else n,
              _p(i0), _p(i1), s2, _p(cb0), _p(cb1), _dt(cb0, "cb0"), _p(scale), _dt(scale, "scale"),
              _p(y), _dt(y, "y"), out, out, n, float(rs), _p(ws), 0 if ws is None else ws.numel(), _stream(dev))
    return y


# ------------------------------------------ sorted copies behind the function entries
# The function-level drop-in (vq_gemv_16 / _16_8 / _16_16, the names a caller
# swaps in for vq2.kernels) has no module to hold a code-sorted copy, so at
# batch 1 it keeps one per index plane of at least SORTED_CACHE_MIN_CODES
# codes, built on the first call (a host repack, ~20 ms for 3 M codes).  An
# entry is used only for the same tensor object (a weak reference: a freed
# plane drops its entry) with an unchanged version counter (an in-place write
# makes a new copy), so a view made anew on every call, or any other plane,
# takes the gather kernel.  The reference's PackedLinear passes its own
# buffers (vq2/runtime.py:93-104), which hit.
SORTED_CACHE_MIN_CODES = 2 << 20
_SORTED_CACHE: dict = {}
_sorted_cache_on = [True]


def sorted_cache_enabled(flag=None) -> bool:
    """Turn the function entries' sorted copies on / off (None: query);
    turning them off drops the copies."""
    if flag is not None:
        _sorted_cache_on[0] = bool(flag)
        if not flag:
            _SORTED_CACHE.clear()
    return _sorted_cache_on[0]


def sorted_cache_bytes() -> int:
    return sum(e[4].nbytes() for e in _SORTED_CACHE.values())


def _cached_sorted(xr, i0, i1, cb0, out, n):
    """The sorted copy of (i0, i1) for a batch-1 call, or None."""
    if not _sorted_cache_on[0] or not i0.is_cuda or cb0.dtype not in (torch.float16, torch.bfloat16):
        return None
    if xr.numel() != n or int(out) * (int(n) // 8) * (1 if i1 is None else 2) < SORTED_CACHE_MIN_CODES:
        return None
    key = id(i0)
    e = _SORTED_CACHE.get(key)
    if (e is not None and e[0]() is i0 and e[1] == i0._version and
            (e[2]() if e[2] is not None else None) is i1 and (i1 is None or e[3] == i1._version)):
        return e[4]
    sp = SortedPlanes(i0, i1, int(out), int(n), device=i0.device)

    def drop(ref, key=key):
        cur = _SORTED_CACHE.get(key)
        if cur is not None and (cur[0] is ref or cur[2] is ref):
            del _SORTED_CACHE[key]

    _SORTED_CACHE[key] = (weakref.ref(i0, drop), i0._version, None if i1 is None else weakref.ref(i1, drop),
                          None if i1 is None else i1._version, sp)
    return sp


def _gemv_entry(xr, i0, i1, cb0, cb1, scale, out, n, rs, out_dtype, y):
    """The reference-named GEMV entries: batch 1 of a large plane on its
    sorted copy (pre-rotated x), otherwise the gather kernel."""
    sp = _cached_sorted(xr, i0, i1, cb0, out, n) if torch.is_tensor(xr) and xr.is_cuda else None
    if sp is not None:
        _dev(xr, i0, i1, cb0, cb1, scale, y)
        if y is not None:
            _contig(y, "y")
            if y.numel() != int(out):
                raise Vq2Error("y has the wrong size")
        yv = None if y is None else y.reshape(-1)
        (r,) = vq_sorted_gemv(_contig(xr, "xr").reshape(-1), [(sp, scale)], cb0, cb1, int(n), hb=0, rs=rs,
                              out_dtype=out_dtype if y is None else y.dtype, ys=None if y is None else [yv])
        return y if y is not None else r.view(*xr.shape[:-1], int(out))
    return vq_gemv(xr, i0, i1, cb0, cb1, scale, out, n, rs, out_dtype=out_dtype, y=y)


def vq_gemv_16(xr, i0, cb0, scale, out, n, rs=1.0, *, out_dtype=torch.bfloat16, y=None):
    """xr [n] -> y [out] for a 2.0 bpw (16,) matrix (vq2/kernels.py:224-230).
    Batch 1 of a plane of >= 2 M codes runs on a code-sorted copy of it (see
    SORTED_CACHE_MIN_CODES)."""
    return _gemv_entry(xr, i0, None, cb0, None, scale, out, n, rs, out_dtype, y)


def vq_gemv_16_8(xr, i0, i1, cb0, cb1, scale, out, n, rs=1.0, *, out_dtype=torch.bfloat16, y=None):
    """xr [n] -> y [out] for a 3.0 bpw (16,8) matrix (vq2/kernels.py:215-221)."""
    if i1.dtype != torch.uint8:
        raise Vq2Error("vq_gemv_16_8: i1 must be uint8")
    return _gemv_entry(xr, i0, i1, cb0, cb1, scale, out, n, rs, out_dtype, y)


def vq_gemv_16_16(xr, i0, i1, cb0, cb1, scale, out, n, rs=1.0, *, out_dtype=torch.bfloat16, y=None):
    """xr [n] -> y [out] for a 4.0 bpw (16,16) matrix: both planes decoded as
    uint16 (the PackedLinear fallback semantics, vq2/runtime.py:82-89)."""
    if i1.dtype == torch.uint8:
        raise Vq2Error("vq_gemv_16_16: i1 must be int16 (uint16 codes)")
    return _gemv_entry(xr, i0, i1, cb0, cb1, scale, out, n, rs, out_dtype, y)


# Largest activation block (batch x n values) whose RHT vq_gemv_rht builds
# inside the GEMV launch: one prologue pass of a 768-thread workgroup.
FUSED_RHT_MAX_VALS = 6144


def vq_gemv_rht(x, mats, cb0, cb1, n, perm=None, sign=None, hb=2048, rht_scale=None, rs=1.0, *,
                out_dtype=torch.float32, ys=None):
    """Rotate x with the RHT and multiply by up to 4 VQ matrices (the q/k/v
    or gate/up fusion of a decoder layer).  B * n <= 6144: one launch, every
    workgroup rotates x in its LDS (one pass of up to 768 threads, overlapped
    with the first gathers); larger blocks: a separate vq_rht launch, then one
    launch of the matrices.  x [n] or [B, n] (B <= 2); mats: list of
    (i0, i1 or None, scale, out_rows) sharing one cfg.  Returns the list of
    outputs ([out] or [B, out])."""
    n = int(n)
    s2, mats = check_gemv_rht_mats(mats, cb0, cb1, n)
    dev = _dev(x, cb0, cb1, perm, sign, *[t for m in mats for t in m[:3]])
    x2 = _contig(x, "x").reshape(-1, n)
    B = x2.shape[0]
    for t, nm, dt in ((perm, "perm", torch.int32), (sign, "sign", torch.int8)):
        if t is not None and (t.dtype != dt or t.numel() != n or not t.is_contiguous()):
            raise Vq2Error(f"{nm} must be a contiguous {dt} [n]")
    if ys is not None and len(ys) != len(mats):
        raise Vq2Error("vq_gemv_rht: one output per matrix")
    segs = (_lib.Seg * len(mats))()
    outs = []
    for k, (i0, i1, scale, out_rows) in enumerate(mats):
        y = ys[k] if ys is not None else torch.empty((B, out_rows) if x.dim() == 2 else (out_rows,),
                                                      dtype=out_dtype, device=dev)
        _contig(y, "y")
        if y.numel() != B * out_rows or y.device != dev:
            raise Vq2Error(f"vq_gemv_rht: output {k} must hold [B, out_rows] = [{B}, {out_rows}] on {dev}")
        segs[k] = _lib.Seg(_p(i0), _p(i1), _p(scale), _p(y), out_rows, out_rows)
        outs.append(y)
    if any(o.dtype != outs[0].dtype for o in outs):
        raise Vq2Error("vq_gemv_rht: the outputs of a launch share a dtype")
    sc = float(hb) ** -0.5 if rht_scale is None else float(rht_scale)
    if B * n > FUSED_RHT_MAX_VALS:
        x2 = vq_rht(x2, perm, sign, hb, sc, out_dtype=torch.float32)
        perm = sign = None
        hb = 0
    _lib.call("vq2_gemv_rht", _p(x2), _dt(x2, "x"), B, n, _p(perm), _p(sign), int(hb), sc, len(mats), segs,
              s2, _p(_contig(cb0, "cb0")), _p(cb1.contiguous()) if cb1 is not None else None, _dt(cb0, "cb0"),
              _dt(mats[0][2], "scale"), _dt(outs[0], "y"), n, float(rs), _stream(dev))
    return outs


# ------------------------------------------------------- code-sorted layout
# uint32 words per iteration of the sorted layout: 64 lanes x 12 bytes, the
# four 64-lane instructions of 63 codes and one base code each
ITER_WORDS = 192


class SortedPlanes:
    """Code-sorted internal layout of one VQ matrix (vq2_sorted_pack): the
    reference's int16 index planes (2 bpw, or the two planes of (16,16)
    4 bpw) repacked once, on the host, into chunks of rows whose codes are
    sorted by value, so that a wave's centroid gathers share codebook lines.
    Built at load time by the modules that own a matrix (PackedLinear,
    PackedLMHead); the planes themselves stay the public format."""

    def __init__(self, i0, i1, out_rows, n, device=None, threads=0, chunk_align=None, rows_per_chunk=None):
        lib = _lib.load()
        n, out_rows = int(n), int(out_rows)
        if n % 8:
            raise Vq2Error(f"n={n} must be a multiple of 8")
        ng = n // 8
        i0 = _idx16(i0, "i0")
        if i0.numel() != out_rows * ng:
            raise Vq2Error(f"i0 has {i0.numel()} codes, expected {out_rows * ng}")
        # stage-2 kind: 0 none, 1 int16 plane ((16,16), 65536-row cb1), 2 uint8
        # plane ((16,8), 256-row cb1: its codes are packed as 16-bit codes
        # below 256, and the kernels mask them to 8 bits)
        self.s2_kind = 0
        if i1 is not None:
            if i1.dtype == torch.uint8:
                _contig(i1, "i1")
                self.s2_kind = 2
            else:
                i1 = _idx16(i1, "i1")
                self.s2_kind = 1
            if i1.numel() != i0.numel():
                raise Vq2Error("i1 and i0 must have the same number of codes")
        dev = torch.device(device) if device is not None else i0.device
        if chunk_align is None:  # whole rounds of chunks over the device's CUs
            chunk_align = _cu_count(dev) if dev.type == "cuda" else 1
        # rows_per_chunk: the library's default (vq2_sorted_rows_per_chunk)
        # unless given; vq2_sorted_pack refuses a height its positions cannot hold
        R = int(lib.vq2_sorted_rows_per_chunk(out_rows, ng, int(chunk_align))) if rows_per_chunk is None \
            else int(rows_per_chunk)
        if R == 0:
            raise Vq2Error(f"sorted layout: n={n} unsupported")
        self.out_rows, self.n, self.rows_per_chunk = out_rows, n, R
        self.n_chunks = -(-out_rows // R)
        self.has_stage2 = i1 is not None
        h0 = i0.detach().to("cpu").contiguous()
        h1 = None if i1 is None else i1.detach().to("cpu").to(torch.int16).contiguous()
        stages = 2 if h1 is not None else 1
        # 252 codes per iteration (lane 63 of an instruction holds its base
        # code), a few instructions more where the packer closes one early
        cap = self.n_chunks * stages * (-(-R * ng // 240) + 8)
        ipc, ipc1, n_iters = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
        for _ in range(2):
            entries = torch.empty(cap * ITER_WORDS, dtype=torch.int32)
            st = lib.vq2_sorted_pack(h0.data_ptr(), None if h1 is None else h1.data_ptr(), out_rows, ng, R,
                                     entries.data_ptr(), cap, ctypes.byref(ipc), ctypes.byref(ipc1),
                                     ctypes.byref(n_iters), int(threads))
            if st == _lib.ERR_ARG and n_iters.value > cap:
                cap = n_iters.value
                continue
            _lib.check(st, "vq2_sorted_pack")
            break
        self.n_iters = int(n_iters.value)
        # every chunk holds iters_per_chunk iterations, stage1_iters of stage 1
        self.iters_per_chunk, self.stage1_iters = int(ipc.value), int(ipc1.value)
        # uint32 entry words held in an int32 tensor (same bits)
        self.entries = entries[: self.n_iters * ITER_WORDS].to(dev)
        self.device = dev

    def mat(self, scale, y=None) -> "_lib.SortedMat":
        _contig(scale, "scale")
        if scale.numel() != self.out_rows:
            raise Vq2Error(f"scale has {scale.numel()} entries, expected {self.out_rows}")
        _dt(scale, "scale")
        return _lib.SortedMat(self.entries.data_ptr(), self.iters_per_chunk, self.stage1_iters, self.n_iters,
                              self.rows_per_chunk, self.s2_kind, scale.data_ptr(), _p(y), self.out_rows)

    def nbytes(self):
        return self.entries.numel() * self.entries.element_size()


_CU_COUNT: dict = {}


def _cu_count(dev: torch.device) -> int:
    if dev.index not in _CU_COUNT:
        _CU_COUNT[dev.index] = torch.cuda.get_device_properties(dev).multi_processor_count
    return _CU_COUNT[dev.index]


def sorted_launch_rows_per_chunk(rows, ng, dev):
    """Chunk height for matrices of `ng` groups sharing one launch (q, k and
    v): launches of fewer than 2^20 codes (stage 1) take about 0.75 x CUs
    chunks over their total rows, at most 64 rows each, one workgroup per
    chunk (the library's rule for one small matrix, applied to the launch);
    None for larger launches (each matrix its own default)."""
    total = sum(int(r) for r in rows)
    if total * int(ng) >= 1 << 20:
        return None
    cu = _cu_count(dev)
    gb = max(0, (int(ng) - 1).bit_length())
    rmax = min((1 << (16 - gb)) - 1, 255) if gb <= 15 else 0  # 16-bit positions
    r = -(-4 * total // (3 * cu))
    return max(1, min(r, 64, rmax))


def sorted_slices(planes, dev) -> int:
    """Workgroups per chunk: as many as keep the launch within one workgroup
    per CU (the per-CU gather rate bounds this kernel, so a CU holding two
    workgroups of one launch finishes last; measured on the gate/up pair:
    50 chunks x 5 slices 20.0 us, x 6 slices 31 us), and few enough that
    each of a workgroup's 16 waves has at least one iteration (measured on
    q, k, v of 2048-wide attention, 15 chunks of 171-228 iterations: 17
    slices 10.6 us, 6-12 slices 9.3 us).  One slice where fewer than three
    fit: the slice sum costs more than the shorter chunk saves (the o
    projection 2048 x 2048: 128 chunks of 16 rows 6.97 us at one slice, 8.1
    at two; 86 chunks of 24 rows 7.28 against 8.06)."""
    chunks = sum(p.n_chunks for p in planes)
    per_wave = min(p.iters_per_chunk for p in planes) // 20
    fit = _cu_count(dev) // chunks
    return max(1, min(32, fit, per_wave)) if fit >= 3 else 1


def _sorted_cbs(planes, cb0, cb1):
    _contig(cb0, "cb0")
    if cb0.dim() != 2 or cb0.shape[0] < 65536 or cb0.shape[1] != 8:
        raise Vq2Error(f"cb0 must be [65536, 8], got {tuple(cb0.shape)}")
    if cb0.dtype not in (torch.float16, torch.bfloat16):
        raise Vq2Error("the sorted layout takes fp16 / bf16 codebooks")
    if any(p.s2_kind != planes[0].s2_kind for p in planes):
        raise Vq2Error("the matrices of a sorted launch share one cfg")
    if planes[0].has_stage2:
        rows = 256 if planes[0].s2_kind == 2 else 65536
        if cb1 is None or cb1.dim() != 2 or cb1.shape[0] < rows or cb1.shape[1] != 8 or cb1.dtype != cb0.dtype:
            raise Vq2Error(f"this matrix needs cb1 [{rows}, 8] in the dtype of cb0")
        _contig(cb1, "cb1")
        return cb0, cb1
    return cb0, None


def _sorted_x(x, n, perm, sign, hb, rht_scale):
    x2 = _contig(x, "x").reshape(-1)
    if x2.numel() != n:
        raise Vq2Error(f"the sorted GEMV takes one activation of n={n} values, got {x2.numel()}")
    hb = int(hb or 0)
    for t, nm, dt in ((perm, "perm", torch.int32), (sign, "sign", torch.int8)):
        if t is not None and (t.dtype != dt or t.numel() != n or not t.is_contiguous()):
            raise Vq2Error(f"{nm} must be a contiguous {dt} [n]")
    sc = (float(hb) ** -0.5 if hb else 1.0) if rht_scale is None else float(rht_scale)
    return x2, hb, sc


def vq_sorted_gemv(x, mats, cb0, cb1, n, perm=None, sign=None, hb=2048, rht_scale=None, rs=1.0, *,
                   out_dtype=torch.float32, ys=None, slices=None):
    """Batch-1 VQ GEMV of up to 4 matrices in the code-sorted layout that
    share one activation: y_m = VQ(W_m) RHT(x) (hb > 0: the rotation is built
    in the kernel's LDS; hb = 0: x is already rotated).  mats: list of
    (SortedPlanes, scale).  With several workgroups (slices) per chunk the
    last of them to finish sums their partials, in slice order, in the same
    launch.  Returns the list of outputs [out_rows]."""
    n = int(n)
    planes = [m[0] for m in mats]
    if not 1 <= len(mats) <= 4 or any(p.n != n for p in planes):
        raise Vq2Error("vq_sorted_gemv: 1..4 matrices of width n")
    if any(p.has_stage2 != planes[0].has_stage2 for p in planes):
        raise Vq2Error("vq_sorted_gemv: the matrices of a launch share one cfg")
    dev = _dev(x, cb0, cb1, perm, sign, *[m[1] for m in mats], *[p.entries for p in planes])
    cb0, cb1 = _sorted_cbs(planes, cb0, cb1)
    x2, hb, sc = _sorted_x(x, n, perm, sign, hb, rht_scale)
    if ys is None:
        ys = [torch.empty(p.out_rows, dtype=out_dtype, device=dev) for p in planes]
    arr = (_lib.SortedMat * len(mats))()
    for k, ((p, s), y) in enumerate(zip(mats, ys)):
        _contig(y, "y")
        if y.numel() != p.out_rows or y.dtype != ys[0].dtype:
            raise Vq2Error(f"vq_sorted_gemv: output {k} must be [{p.out_rows}] of the launch's dtype")
        if s.dtype != mats[0][1].dtype:
            raise Vq2Error("vq_sorted_gemv: the scales of a launch share a dtype")
        arr[k] = p.mat(s, y)
    slices = sorted_slices(planes, dev) if slices is None else int(slices)
    lib = _lib.load()
    ws = _workspace(dev, int(lib.vq2_sorted_gemv_workspace(arr, len(mats), slices)), sorted_kind=True)
    _lib.call("vq2_sorted_gemv", _p(x2), _dt(x2, "x"), _p(perm), _p(sign), hb, sc, len(mats), arr, _p(cb0), _p(cb1),
              _dt(cb0, "cb0"), _dt(mats[0][1], "scale"), _dt(ys[0], "y"), n, float(rs), slices, _p(ws),
              0 if ws is None else ws.numel(), _stream(dev))
    return ys


def vq_sorted_gemv_argmax(x, planes, scale, cb0, cb1, n, perm=None, sign=None, hb=0, rht_scale=None, rs=1.0):
    """LM head + top-1 at batch 1 over a code-sorted matrix: (idx int64 [1],
    val fp32 [1]), torch.argmax's first maximum of the logits, which are
    never written."""
    n = int(n)
    if planes.n != n:
        raise Vq2Error("vq_sorted_gemv_argmax: planes of another width")
    dev = _dev(x, cb0, cb1, perm, sign, scale, planes.entries)
    cb0, cb1 = _sorted_cbs([planes], cb0, cb1)
    x2, hb, sc = _sorted_x(x, n, perm, sign, hb, rht_scale)
    lib = _lib.load()
    m = planes.mat(scale)
    ws = _workspace(dev, int(lib.vq2_sorted_gemv_argmax_workspace(ctypes.byref(m))))
    idx = torch.empty(1, dtype=torch.int64, device=dev)
    val = torch.empty(1, dtype=torch.float32, device=dev)
    _lib.call("vq2_sorted_gemv_argmax", _p(x2), _dt(x2, "x"), _p(perm), _p(sign), hb, sc, ctypes.byref(m), _p(cb0),
              _p(cb1), _dt(cb0, "cb0"), _dt(scale, "scale"), n, float(rs), _p(ws), ws.numel(), _p(idx), _p(val),
              _stream(dev))
    return idx, val


SORTED_BATCH_MAX = 4


def sorted_batch_slices(planes, dev) -> int:
    """Workgroups per chunk of the batch 2-4 launch (8-wave workgroups, two
    per CU): as many as keep the launch within one round, and few enough
    that each wave has at least one iteration."""
    chunks = sum(p.n_chunks for p in planes)
    per_wave = min(p.iters_per_chunk for p in planes) // 10
    return max(1, min(32, 2 * _cu_count(dev) // chunks, per_wave))


def sorted_batch_fits(planes, batch) -> bool:
    """Whether the batch kernel's LDS (fp16 activation of 2 or 4 rows, and
    the accumulators of the tallest chunk) fits its 150 KiB (two workgroups
    per CU up to 80 KiB): n = 2048 with any chunk height, n = 6144 with the
    default 62-row chunks.  Batch 3-4 whose 4-row workgroups would exceed
    80 KiB runs as launches of at most 2 rows, so those must fit."""
    n = planes[0].n
    # 8 waves x 2 accumulator arrays per row (4 for chunks of at most 32 rows)
    acc = max((32 if p.rows_per_chunk <= 32 else 16) * (p.rows_per_chunk + 1) for p in planes)
    shm = lambda nb: (max(n * nb // 2, 512 * nb) + acc * nb) * 4
    if batch > 2 and shm(4) <= 80 * 1024:
        return True
    return shm(2) <= 150 * 1024


def _batch_x(x, n):
    x2 = _contig(x, "x").reshape(-1, n)
    if not 1 <= x2.shape[0] <= SORTED_BATCH_MAX:
        raise Vq2Error(f"the sorted batch kernels take 1..{SORTED_BATCH_MAX} activation rows, got {x2.shape[0]}")
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    return x2


def vq_sorted_gemm_batch(x, mats, cb0, cb1, n, rs=1.0, *, out_dtype=torch.float32, ys=None, slices=None):
    """VQ GEMM of B = 1..4 rotated activation rows x [B, n] with up to 4
    code-sorted matrices: one centroid gather serves every row (the
    activation is held in fp16 with a power-of-two scale per row).  mats:
    list of (SortedPlanes, scale).  Returns the list of outputs [B, out_rows]."""
    n = int(n)
    planes = [m[0] for m in mats]
    if not 1 <= len(mats) <= 4 or any(p.n != n for p in planes):
        raise Vq2Error("vq_sorted_gemm_batch: 1..4 matrices of width n")
    if any(p.has_stage2 != planes[0].has_stage2 for p in planes):
        raise Vq2Error("vq_sorted_gemm_batch: the matrices of a launch share one cfg")
    dev = _dev(x, cb0, cb1, *[m[1] for m in mats], *[p.entries for p in planes])
    cb0, cb1 = _sorted_cbs(planes, cb0, cb1)
    x2 = _batch_x(x, n)
    B = x2.shape[0]
    if ys is None:
        ys = [torch.empty((B, p.out_rows), dtype=out_dtype, device=dev) for p in planes]
    arr = (_lib.SortedMat * len(mats))()
    for k, ((p, s), y) in enumerate(zip(mats, ys)):
        _contig(y, "y")
        if y.numel() != B * p.out_rows or y.dtype != ys[0].dtype or y.device != dev:
            raise Vq2Error(f"vq_sorted_gemm_batch: output {k} must be [{B}, {p.out_rows}] of the launch's dtype")
        if s.dtype != mats[0][1].dtype:
            raise Vq2Error("vq_sorted_gemm_batch: the scales of a launch share a dtype")
        arr[k] = p.mat(s, y)
    slices = sorted_batch_slices(planes, dev) if slices is None else int(slices)
    lib = _lib.load()
    ws = _workspace(dev, int(lib.vq2_sorted_gemm_batch_workspace(arr, len(mats), B, slices)), sorted_kind=True)
    _lib.call("vq2_sorted_gemm_batch", _p(x2), _dt(x2, "x"), B, n, len(mats), arr, _p(cb0), _p(cb1),
              _dt(cb0, "cb0"), _dt(mats[0][1], "scale"), _dt(ys[0], "y"), n, float(rs), slices, _p(ws),
              0 if ws is None else ws.numel(), _stream(dev))
    return ys


def vq_sorted_gemm_batch_argmax(x, planes, scale, cb0, cb1, n, rs=1.0):
    """LM head + top-1 of B = 1..4 rotated activation rows x [B, n] over a
    code-sorted matrix: (idx int64 [B], val fp32 [B]), torch.argmax's first
    maximum per row of the logits, which are never written."""
    n = int(n)
    if planes.n != n:
        raise Vq2Error("vq_sorted_gemm_batch_argmax: planes of another width")
    dev = _dev(x, cb0, cb1, scale, planes.entries)
    cb0, cb1 = _sorted_cbs([planes], cb0, cb1)
    x2 = _batch_x(x, n)
    B = x2.shape[0]
    lib = _lib.load()
    m = planes.mat(scale)
    ws = _workspace(dev, int(lib.vq2_sorted_gemm_batch_argmax_workspace(ctypes.byref(m), B)))
    idx = torch.empty(B, dtype=torch.int64, device=dev)
    val = torch.empty(B, dtype=torch.float32, device=dev)
    _lib.call("vq2_sorted_gemm_batch_argmax", _p(x2), _dt(x2, "x"), B, n, ctypes.byref(m), _p(cb0), _p(cb1),
              _dt(cb0, "cb0"), _dt(scale, "scale"), n, float(rs), _p(ws), ws.numel(), _p(idx), _p(val),
              _stream(dev))
    return idx, val


# ------------------------------------------------ MoE over sorted expert pools
class SortedPool:
    """Code-sorted layout of an expert pool idx [E, rows, n/8] (int16 stage-1
    plane) with an optional stage-2 plane idx1 of the same shape (int16 for
    (16,16), uint8 for the (16,8) 3 bpw experts; vq2_sorted_pack_pool): every
    expert packed like a SortedPlanes matrix with one chunk height, experts
    one after another, every chunk padded to the same iteration counts (so
    the kernels compute a chunk's offset instead of reading it).  Built once
    at load time by the expert modules; the pool stays the public format.
    ``SortedPool.slots`` makes an empty (zeroed) pool of the same layout for
    a paged slot pool whose records are copied in later.  rows_per_chunk:
    the chunk height (default: vq2_sorted_rows_per_chunk, at most 255 rows);
    up to 511 where 16-bit positions hold it (taller chunks put more codes
    on each code value: fewer codebook lines per instruction, fewer
    workgroups per expert)."""

    def __init__(self, idx, device=None, threads=0, idx1=None, rows_per_chunk=None):
        lib = _lib.load()
        idx = _idx16(idx, "idx")
        if idx.dim() != 3:
            raise Vq2Error(f"expert pool must be [E, rows, ng], got {tuple(idx.shape)}")
        E, rows, ng = (int(v) for v in idx.shape)
        self.s2_kind = 0
        h1 = None
        if idx1 is not None:
            if tuple(idx1.shape) != tuple(idx.shape):
                raise Vq2Error(f"idx1 must be {tuple(idx.shape)}, got {tuple(idx1.shape)}")
            self.s2_kind = 2 if idx1.dtype == torch.uint8 else 1
            if self.s2_kind == 1:
                idx1 = _idx16(idx1, "idx1")
            h1 = idx1.detach().to("cpu").to(torch.int16).contiguous()
        R = int(lib.vq2_sorted_rows_per_chunk(rows, ng, 1))
        if R == 0:
            raise Vq2Error(f"sorted layout: ng={ng} unsupported")
        if rows_per_chunk is not None:
            R = int(rows_per_chunk)  # vq2_sorted_pack_pool checks it against the position bits
        self.n_experts, self.rows, self.ng, self.rows_per_chunk = E, rows, ng, R
        self.chunks = -(-rows // R)
        dev = torch.device(device) if device is not None else idx.device
        h = idx.detach().to("cpu").contiguous()
        stages = 2 if h1 is not None else 1
        cap = E * self.chunks * stages * (-(-R * ng // 240) + 8)
        ipc, ipc1, n_iters = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
        for _ in range(2):
            entries = torch.empty(cap * ITER_WORDS, dtype=torch.int32)
            st = lib.vq2_sorted_pack_pool(h.data_ptr(), None if h1 is None else h1.data_ptr(), E, rows, ng, R,
                                          entries.data_ptr(), cap, ctypes.byref(ipc), ctypes.byref(ipc1),
                                          ctypes.byref(n_iters), int(threads))
            if st == _lib.ERR_ARG and n_iters.value > cap:
                cap = n_iters.value
                continue
            _lib.check(st, "vq2_sorted_pack_pool")
            break
        self.n_iters = int(n_iters.value)
        self.iters_per_chunk, self.stage1_iters = int(ipc.value), int(ipc1.value)
        self.entries = entries[: self.n_iters * ITER_WORDS].to(dev)
        self.device = dev

    @classmethod
    def slots(cls, like: "SortedPool", capacity: int, device=None):
        """An empty pool of `capacity` experts in the layout of `like` (the
        same chunking and iteration counts), zeroed: entry words that decode
        to code 0 at row 0, group 0 of every chunk, so a slot read before its
        record arrives gives finite values, never an out-of-range access."""
        self = cls.__new__(cls)
        for k in ("rows", "ng", "rows_per_chunk", "chunks", "iters_per_chunk", "stage1_iters", "s2_kind"):
            setattr(self, k, getattr(like, k))
        self.n_experts = int(capacity)
        self.n_iters = self.n_experts * self.chunks * self.iters_per_chunk
        dev = torch.device(device) if device is not None else like.device
        self.entries = torch.zeros(self.n_iters * ITER_WORDS, dtype=torch.int32, device=dev)
        self.device = dev
        return self

    def expert_words(self):
        """uint32 words of one expert's chunks (the unit a slot copy moves)."""
        return self.chunks * self.iters_per_chunk * ITER_WORDS

    @property
    def has_stage2(self):
        return self.s2_kind != 0

    def pool(self, scale, cb1=None) -> "_lib.SortedPool":
        _contig(scale, "scale")
        if scale.numel() != self.n_experts * self.rows:
            raise Vq2Error(f"scale must hold [{self.n_experts}, {self.rows}] values")
        if self.s2_kind:
            rows = 256 if self.s2_kind == 2 else 65536
            if cb1 is None or cb1.dim() != 2 or cb1.shape[0] < rows or cb1.shape[1] != 8:
                raise Vq2Error(f"a two-stage pool needs its stage-2 codebook [{rows}, 8]")
            _contig(cb1, "cb1")
        return _lib.SortedPool(self.entries.data_ptr(), self.iters_per_chunk, self.n_iters, self.rows_per_chunk,
                               self.rows, self.ng, scale.data_ptr(), _dt(scale, "scale"), self.stage1_iters,
                               self.s2_kind, _p(cb1) if self.s2_kind else None)

    def nbytes(self):
        return self.entries.numel() * self.entries.element_size()


# per-workgroup rates that set the slice counts below (MI355X, 16-wave
# workgroups): codes per microsecond, and the fixed cost of a workgroup
# (prologue, epilogue) in microseconds
_MOE_RATE = 1460.0
_MOE_FIXED_US = (2.5, 2.0)


def moe_slices(units, codes_per_unit, cu, fixed_us, one_launch=False):
    """Slices per chunk for `units` (pair, chunk) units: the count that
    minimises rounds x (work per slice + fixed cost), with one 16-wave
    workgroup per CU at a time.  one_launch (gate_up and down in one launch,
    two workgroups per CU): units that fill twice the CUs on their own take
    one slice, units that fill the CUs two (measured, T = 8, 360 gate_up and
    648 down units: gate_up / down slices 1 / 1 66.8 us per layer, 2 / 1
    64.5, 3 / 1 64.5, 2 / 2 65.9, 1 / 2 70.5; with the down pool in 5
    taller chunks, 360 and 360 units: 2 / 2 59.0-59.8, 2 / 3 61.2, 3 / 1
    63.2, 3 / 2 63.5, 1 / 1 63.9, 3 / 3 63.9, 1 / 2 64.1, 2 / 1 65.5, 1 / 3
    67.0)."""
    if one_launch and units >= 2 * cu:
        return 1
    if one_launch and units >= cu:
        return 2
    best, best_t = 1, None
    for s in range(1, 33):
        t = -(-units * s // cu) * (codes_per_unit / _MOE_RATE / s + fixed_us)
        if best_t is None or t < best_t - 1e-9:
            best, best_t = s, t
    return best


def _rot_tables(rot, n, what):
    """A rotation (perm int32 [n] or None, sign int8 [n] or None, hb, scale)
    checked for the kernels, which read n entries of each table."""
    if len(rot) != 4:
        raise Vq2Error(f"{what} must be (perm, sign, hb, scale)")
    perm, sign, hb, sc = rot
    _perm_sign(perm, sign, n, what + " ")
    return _lib.RotTables(_p(perm), _p(sign), int(hb), float(sc))


def vq_sorted_moe(h, gate_up: SortedPool, gu_scale, down: SortedPool, dn_scale, cb, rot_h, rot_i, *, ids=None,
                  w=None, logits=None, top_k=None, shared_id=None, shared_gate=None, out_dtype=torch.float32,
                  out=None, slices=None, cb1=None):
    """The experts of an MoE layer over code-sorted pools, two launches
    (gate_up and down in one, then the combine; three at other widths or
    above 127 pairs); a one-launch wait that gives up leaves its pair NaN
    and a bit in vq_sorted_moe_status():
    out [T, H] = sum_k w[t, k] * VQ(down[e]) RHT_I(silu(gu[:I]) * gu[I:]),
    gu = VQ(gate_up[e]) RHT_H(h_t), e = ids[t, k].  With `logits` [T, E_r]
    the router is built in (top_k routed experts plus the shared expert
    shared_id with sigmoid(shared_gate . h_t)); it then returns
    (out, ids int32 [T, top_k + 1], w fp32 [T, top_k + 1]).  rot_h / rot_i:
    (perm int32, sign int8, hb, scale).  Two-stage pools (the (16,8) 3 bpw
    experts) take their stage-2 codebook cb1 ([256, 8] in cb's dtype)."""
    H = gate_up.ng * 8
    I = down.ng * 8
    if gate_up.rows != 2 * I or down.rows != H or gate_up.n_experts != down.n_experts:
        raise Vq2Error("vq_sorted_moe: inconsistent gate_up / down pools")
    h2 = _contig(h, "h").reshape(-1, H)
    T = h2.shape[0]
    rh = _rot_tables(rot_h, H, "rot_h")
    ri = _rot_tables(rot_i, I, "rot_i")
    if logits is not None:
        if shared_gate is None or shared_id is None or top_k is None:
            raise Vq2Error("vq_sorted_moe: the built-in router needs top_k, shared_id and shared_gate")
        _gate_vec(shared_gate, H)
    dev = _dev(h2, cb, gu_scale, dn_scale, ids, w, logits, gate_up.entries, down.entries, rot_h[0], rot_h[1],
               rot_i[0], rot_i[1], shared_gate if logits is not None else None, cb1)
    _contig(cb, "cb")
    if cb.dim() != 2 or cb.shape[0] < 65536 or cb.shape[1] != 8 or cb.dtype not in (torch.float16, torch.bfloat16):
        raise Vq2Error("vq_sorted_moe: cb must be an fp16 / bf16 [65536, 8] codebook")
    router = logits is not None
    if router:
        lg = _contig(logits, "logits").reshape(T, -1)
        P = int(top_k) + 1
        ids_out = torch.empty((T, P), dtype=torch.int32, device=dev)
        w_out = torch.empty((T, P), dtype=torch.float32, device=dev)
        ids_p, ids64, w_p = None, 0, None
    else:
        if ids is None or w is None:
            raise Vq2Error("vq_sorted_moe: ids and w, or router logits, are required")
        ids2 = _contig(ids, "ids").reshape(T, -1)
        if ids2.dtype not in (torch.int32, torch.int64):
            raise Vq2Error("ids must be int32 or int64")
        P = ids2.shape[1]
        w2 = _contig(w, "w").reshape(T, P)
        if w2.dtype != torch.float32:
            raise Vq2Error("w must be fp32")
        ids_p, ids64, w_p = _p(ids2), 1 if ids2.dtype == torch.int64 else 0, _p(w2)
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype, device=dev)
    elif out.numel() != T * H or not out.is_contiguous():
        raise Vq2Error(f"out must be a contiguous [{T}, {H}]")
    if slices is None:
        cu = _cu_count(dev)
        # the library runs gate_up and down as one launch for these shapes
        # (2048-point and 512-point rotations, at most 128 pairs)
        one = H == 2048 and I == 512 and int(rot_h[2]) == 2048 and int(rot_i[2]) == 512 and T * P <= 127
        st = 2 if gate_up.has_stage2 else 1
        sg = moe_slices(T * P * gate_up.chunks, st * gate_up.rows_per_chunk * gate_up.ng, cu, _MOE_FIXED_US[0], one)
        sd = moe_slices(T * P * down.chunks, st * down.rows_per_chunk * down.ng, cu, _MOE_FIXED_US[1], one)
    else:
        sg, sd = (int(v) for v in slices)
    lib = _lib.load()
    ws = _workspace(dev, int(lib.vq2_sorted_moe_workspace(T, P, H, I, sg, sd)), sorted_kind=True)
    if cb1 is not None and cb1.dtype != cb.dtype:
        raise Vq2Error("vq_sorted_moe: cb1 must have cb's dtype")
    gp, dp = gate_up.pool(gu_scale, cb1), down.pool(dn_scale, cb1)
    _lib.call("vq2_sorted_moe", _p(h2), _dt(h2, "h"), T, P, ids_p, ids64, w_p,
              _p(lg) if router else None, _dt(lg, "logits") if router else 0, lg.shape[1] if router else 0,
              int(top_k) if router else 0, int(shared_id) if router else 0, _p(shared_gate) if router else None,
              _dt(shared_gate, "shared_gate") if router else 0, _p(ids_out) if router else None,
              _p(w_out) if router else None, gate_up.n_experts, H, I, ctypes.byref(gp), ctypes.byref(dp), _p(cb),
              _dt(cb, "cb"), ctypes.byref(rh), ctypes.byref(ri), _p(out), _dt(out, "out"), sg, sd, _p(ws),
              ws.numel(), _stream(dev))
    if router:
        return out, ids_out, w_out
    return out


# -------------------------------------------------------------- grouped MoE
def _moe_checks(pool, scale, OUT, NG, what):
    pool = _idx16(pool, what)
    if pool.dim() != 3 or pool.shape[1] != OUT or pool.shape[2] != NG:
        raise Vq2Error(f"{what}: pool must be [E, {OUT}, {NG}], got {tuple(pool.shape)}")
    _contig(scale, "scale")
    if scale.numel() != pool.shape[0] * OUT:
        raise Vq2Error(f"{what}: scale must be [E, {OUT}]")
    return pool


def vq_moe_parallel_gate_up(xr, topk_ids, gate_up_idx, cb16, gate_up_scale, y_out, OUT=1024, NG=256, rs=1.0):
    """y_out[k, :OUT] = VQ(pool[topk_ids[k]]) xr for every k (x shared).
    Writes y_out in place, returns None (vq2/kernels.py:246-254)."""
    dev = _dev(xr, topk_ids, gate_up_idx, cb16, gate_up_scale, y_out)
    OUT, NG = int(OUT), int(NG)
    pool = _moe_checks(gate_up_idx, gate_up_scale, OUT, NG, "gate_up_idx")
    ids, ids_dt = _ids(topk_ids)
    K = ids.numel()
    x = _contig(xr, "xr").reshape(-1)
    if x.numel() < NG * 8:
        raise Vq2Error(f"xr has {x.numel()} values, need {NG * 8}")
    if y_out.dim() != 2 or y_out.shape[0] < K or y_out.shape[1] < OUT or y_out.stride(1) != 1:
        raise Vq2Error("y_out must be [>=K, >=OUT] with unit column stride")
    _contig(cb16, "cb16")
    _lib.call("vq2_moe_grouped", _p(x), _dt(x, "xr"), 0, 1, _p(ids), ids_dt, K, _p(pool), pool.shape[0],
              _p(cb16), _dt(cb16, "cb16"), _p(gate_up_scale), _dt(gate_up_scale, "scale"),
              _p(y_out), _dt(y_out, "y_out"), y_out.stride(0), OUT, NG, float(rs), _stream(dev))


def vq_moe_parallel_down(act_r, topk_ids, down_idx, cb16, down_scale, y_out, OUT=2048, NG=64, rs=1.0):
    """y_out[k, :OUT] = VQ(pool[topk_ids[k]]) act_r[k] (one activation per
    expert).  Writes y_out in place, returns None (vq2/kernels.py:256-264)."""
    dev = _dev(act_r, topk_ids, down_idx, cb16, down_scale, y_out)
    OUT, NG = int(OUT), int(NG)
    pool = _moe_checks(down_idx, down_scale, OUT, NG, "down_idx")
    ids, ids_dt = _ids(topk_ids)
    K = ids.numel()
    a = _contig(act_r, "act_r").reshape(-1)
    if a.numel() < K * NG * 8:
        raise Vq2Error(f"act_r has {a.numel()} values, need K*NG*8 = {K * NG * 8}")
    if y_out.dim() != 2 or y_out.shape[0] < K or y_out.shape[1] < OUT or y_out.stride(1) != 1:
        raise Vq2Error("y_out must be [>=K, >=OUT] with unit column stride")
    _contig(cb16, "cb16")
    _lib.call("vq2_moe_grouped", _p(a), _dt(a, "act_r"), NG * 8, 1, _p(ids), ids_dt, K, _p(pool), pool.shape[0],
              _p(cb16), _dt(cb16, "cb16"), _p(down_scale), _dt(down_scale, "scale"),
              _p(y_out), _dt(y_out, "y_out"), y_out.stride(0), OUT, NG, float(rs), _stream(dev))


def vq_moe_grouped(x, ids, pool, cb16, pool_scale, y_out, OUT, NG, rs=1.0, pairs_per_x=1, shared_x=False):
    """General grouped launch: y_out[k] = VQ(pool[ids.flat[k]]) x_k with
    x_k = x[k // pairs_per_x] (or x itself for every k when shared_x)."""
    dev = _dev(x, ids, pool, cb16, pool_scale, y_out)
    OUT, NG = int(OUT), int(NG)
    pool = _moe_checks(pool, pool_scale, OUT, NG, "pool")
    ids2, ids_dt = _ids(ids)
    K = ids2.numel()
    xx = _contig(x, "x").reshape(-1)
    need = NG * 8 if shared_x else ((K + pairs_per_x - 1) // pairs_per_x) * NG * 8
    if xx.numel() < need:
        raise Vq2Error(f"x has {xx.numel()} values, need {need}")
    y2 = y_out.reshape(-1, y_out.shape[-1]) if y_out.dim() != 2 else y_out
    if y2.shape[0] < K or y2.shape[1] < OUT or y2.stride(1) != 1:
        raise Vq2Error("y_out must be [>=K, >=OUT] with unit column stride")
    _contig(cb16, "cb16")
    _lib.call("vq2_moe_grouped", _p(xx), _dt(xx, "x"), 0 if shared_x else NG * 8, int(pairs_per_x), _p(ids2),
              ids_dt, K, _p(pool), pool.shape[0], _p(cb16), _dt(cb16, "cb16"), _p(pool_scale),
              _dt(pool_scale, "scale"), _p(y2), _dt(y2, "y_out"), y2.stride(0), OUT, NG, float(rs), _stream(dev))
    return y_out


def _stage2_pool(pool, pool1, cb16, cb8):
    """uint8 stage-2 plane of a (16,8) expert pool: same [E, rows, ng] shape
    as the int16 stage-1 pool; cb8 [256, 8] in the dtype of cb16."""
    if pool1 is None and cb8 is None:
        return None, None
    if pool1 is None or cb8 is None:
        raise Vq2Error("a (16,8) pool needs both pool1 and cb8")
    p1 = _contig(pool1, "pool1")
    if p1.dtype != torch.uint8 or tuple(p1.shape) != tuple(pool.shape):
        raise Vq2Error(f"pool1 must be uint8 {tuple(pool.shape)}, got {p1.dtype} {tuple(p1.shape)}")
    c8 = _contig(cb8, "cb8")
    if tuple(c8.shape) != (256, 8) or c8.dtype != cb16.dtype:
        raise Vq2Error(f"cb8 must be [256, 8] {cb16.dtype}")
    return p1, c8


def vq_moe_gate_up_rht(h, ids, pool, cb16, pool_scale, y_out, OUT, NG, perm=None, sign=None, hb=2048,
                       rht_scale=None, rs=1.0, pool1=None, cb8=None):
    """Grouped gate_up with the activation RHT fused: token t = row of h
    [T, NG*8], experts ids [T, P]; y_out [T*P, >=OUT].  pool1 / cb8 select a
    (16,8) pool: uint8 stage-2 codes [E, OUT, NG] and their [256, 8]
    codebook (promoted 3 bpw experts)."""
    dev = _dev(h, ids, pool, cb16, pool_scale, y_out, perm, sign, pool1, cb8)
    OUT, NG = int(OUT), int(NG)
    pool = _moe_checks(pool, pool_scale, OUT, NG, "pool")
    ids2, ids_dt = _ids(ids)
    if ids2.dim() != 2:
        raise Vq2Error("ids must be [T, P]")
    T, P = ids2.shape
    hh = _contig(h, "h").reshape(-1, NG * 8)
    if hh.shape[0] != T:
        raise Vq2Error("h must be [T, NG*8]")
    _perm_sign(perm, sign, NG * 8)
    y2 = y_out.reshape(-1, y_out.shape[-1])
    if y2.shape[0] < T * P or y2.shape[1] < OUT or y2.stride(1) != 1:
        raise Vq2Error("y_out must be [>=T*P, >=OUT] with unit column stride")
    sc = float(hb) ** -0.5 if rht_scale is None else float(rht_scale)
    p1, c8 = _stage2_pool(pool, pool1, cb16, cb8)
    if p1 is None:
        _lib.call("vq2_moe_gate_up_rht", _p(hh), _dt(hh, "h"), T, _p(perm), _p(sign), int(hb), sc, _p(ids2), ids_dt,
                  P, _p(pool), pool.shape[0], _p(_contig(cb16, "cb16")), _dt(cb16, "cb16"), _p(pool_scale),
                  _dt(pool_scale, "scale"), _p(y2), _dt(y2, "y_out"), y2.stride(0), OUT, NG, float(rs), _stream(dev))
    else:
        _lib.call("vq2_moe_gate_up_rht_16_8", _p(hh), _dt(hh, "h"), T, _p(perm), _p(sign), int(hb), sc, _p(ids2),
                  ids_dt, P, _p(pool), _p(p1), pool.shape[0], _p(_contig(cb16, "cb16")), _p(c8), _dt(cb16, "cb16"),
                  _p(pool_scale), _dt(pool_scale, "scale"), _p(y2), _dt(y2, "y_out"), y2.stride(0), OUT, NG,
                  float(rs), _stream(dev))
    return y_out


def vq_moe_router_gate_up_rht(h, router_logits, top_k, pool, cb16, pool_scale, y_out, OUT, NG, shared_gate=None,
                              shared_id=-1, perm=None, sign=None, hb=2048, rht_scale=None, rs=1.0):
    """Router + grouped gate_up + activation RHT in one launch: token t = row
    of h [T, NG*8], logits [T, E]; P = top_k (+1 with a shared expert).
    y_out [T*P, >=OUT].  Returns (ids int32 [T, P], w fp32 [T, P]) exactly
    as vq_router_topk for the down/combine launch."""
    dev = _dev(h, router_logits, pool, cb16, pool_scale, y_out, perm, sign, shared_gate)
    OUT, NG, k = int(OUT), int(NG), int(top_k)
    pool = _moe_checks(pool, pool_scale, OUT, NG, "pool")
    lg = _contig(router_logits, "router_logits")
    hh = _contig(h, "h").reshape(-1, NG * 8)
    T = hh.shape[0]
    lg2 = lg.reshape(T, -1)
    P = k + (1 if shared_id >= 0 else 0)
    y2 = y_out.reshape(-1, y_out.shape[-1])
    if y2.shape[0] < T * P or y2.shape[1] < OUT or y2.stride(1) != 1:
        raise Vq2Error("y_out must be [>=T*P, >=OUT] with unit column stride")
    ids = torch.empty((T, P), dtype=torch.int32, device=dev)
    w = torch.empty((T, P), dtype=torch.float32, device=dev)
    _perm_sign(perm, sign, NG * 8)
    if shared_id >= 0 and shared_gate is None:
        raise Vq2Error("a shared expert needs shared_gate")
    sg = _gate_vec(shared_gate, NG * 8) if shared_gate is not None else None
    sc = float(hb) ** -0.5 if rht_scale is None else float(rht_scale)
    _lib.call("vq2_moe_router_gate_up_rht", _p(hh), _dt(hh, "h"), T, _p(perm), _p(sign), int(hb), sc,
              _p(lg2), _dt(lg2, "router_logits"), lg2.shape[1], k, _p(sg), _dt(sg, "shared_gate") if sg is not None else 0,
              int(shared_id), _p(pool), pool.shape[0], _p(_contig(cb16, "cb16")), _dt(cb16, "cb16"), _p(pool_scale),
              _dt(pool_scale, "scale"), _p(y2), _dt(y2, "y_out"), y2.stride(0), OUT, NG, float(rs), _p(ids), _p(w),
              _stream(dev))
    return ids, w


def vq_moe_down_swiglu_combine(gu, ids, w, down_idx, cb16, down_scale, OUT, NG, perm=None, sign=None, hb=None,
                               rht_scale=None, rs=1.0, out=None, out_dtype=torch.float32, pool1=None, cb8=None,
                               accumulate=False):
    """silu(gate)*up -> RHT -> grouped down -> weighted combine, one launch.
    gu [T*P, >=2*NG*8] (gate | up), ids [T, P], w fp32 [T, P] -> out [T, OUT].
    pool1 / cb8: (16,8) pool as in vq_moe_gate_up_rht; accumulate adds the
    combine to the given out (the (16,8) entry only)."""
    dev = _dev(gu, ids, w, down_idx, cb16, down_scale, out, perm, sign, pool1, cb8)
    OUT, NG = int(OUT), int(NG)
    pool = _moe_checks(down_idx, down_scale, OUT, NG, "down_idx")
    ids2, ids_dt = _ids(ids)
    if ids2.dim() != 2:
        raise Vq2Error("ids must be [T, P]")
    T, P = ids2.shape
    if w.dtype != torch.float32 or w.numel() != T * P:
        raise Vq2Error("w must be float32 [T, P]")
    _contig(w, "w")
    g2 = gu.reshape(-1, gu.shape[-1])
    if g2.shape[0] != T * P or g2.shape[1] < 2 * NG * 8 or g2.stride(1) != 1:
        raise Vq2Error("gu must be [T*P, >=2*NG*8] with unit column stride")
    _perm_sign(perm, sign, NG * 8)
    hb = NG * 8 if hb is None else int(hb)
    sc = float(hb) ** -0.5 if rht_scale is None else float(rht_scale)
    p1, c8 = _stage2_pool(pool, pool1, cb16, cb8)
    if accumulate and (out is None or p1 is None):
        raise Vq2Error("accumulate needs an out tensor and a (16,8) pool")
    if out is None:
        out = torch.empty((T, OUT), dtype=out_dtype, device=dev)
    _contig(out, "out")
    if out.numel() < T * OUT:
        raise Vq2Error(f"out must hold [T, OUT] = [{T}, {OUT}]")
    if p1 is None:
        _lib.call("vq2_moe_down_swiglu_combine", _p(g2), _dt(g2, "gu"), g2.stride(0), _p(perm), _p(sign), hb, sc,
                  _p(ids2), ids_dt, _p(w), T, P, _p(pool), pool.shape[0], _p(_contig(cb16, "cb16")),
                  _dt(cb16, "cb16"), _p(down_scale), _dt(down_scale, "scale"), _p(out), _dt(out, "out"), OUT, OUT, NG,
                  float(rs), _stream(dev))
    else:
        _lib.call("vq2_moe_down_swiglu_combine_16_8", _p(g2), _dt(g2, "gu"), g2.stride(0), _p(perm), _p(sign), hb,
                  sc, _p(ids2), ids_dt, _p(w), T, P, _p(pool), _p(p1), pool.shape[0], _p(_contig(cb16, "cb16")),
                  _p(c8), _dt(cb16, "cb16"), _p(down_scale), _dt(down_scale, "scale"), _p(out), _dt(out, "out"), OUT,
                  OUT, NG, float(rs), 1 if accumulate else 0, _stream(dev))
    return out


def vq_moe_down_combine(act_r, ids, w, down_idx, cb16, down_scale, out=None, OUT=2048, NG=64, rs=1.0,
                        out_dtype=torch.float32):
    """Grouped down projection fused with the weighted combine.
    act_r [T*P, NG*8], ids [T, P], w fp32 [T, P] -> out [T, OUT] with
    out[t] = sum_j w[t, j] * VQ(pool[ids[t, j]]) act_r[t*P + j]."""
    dev = _dev(act_r, ids, w, down_idx, cb16, down_scale, out)
    OUT, NG = int(OUT), int(NG)
    pool = _moe_checks(down_idx, down_scale, OUT, NG, "down_idx")
    ids2, ids_dt = _ids(ids)
    if ids2.dim() != 2:
        raise Vq2Error("ids must be [T, P]")
    T, P = ids2.shape
    if w.dtype != torch.float32 or w.numel() != T * P:
        raise Vq2Error("w must be float32 [T, P]")
    _contig(w, "w")
    a = _contig(act_r, "act_r")
    if a.numel() != T * P * NG * 8:
        raise Vq2Error("act_r must be [T*P, NG*8]")
    if out is None:
        out = torch.empty((T, OUT), dtype=out_dtype, device=dev)
    _contig(out, "out")
    _lib.call("vq2_moe_down_combine", _p(a), _dt(a, "act_r"), _p(ids2), ids_dt, _p(w), T, P, _p(pool),
              pool.shape[0], _p(cb16), _dt(cb16, "cb16"), _p(down_scale), _dt(down_scale, "scale"),
              _p(out), _dt(out, "out"), OUT, OUT, NG, float(rs), _stream(dev))
    return out


# --------------------------------------------------------------------- RHT
def vq_rht(x, perm=None, sign=None, hb=2048, scale=None, inverse=False, *, out=None, out_dtype=None):
    """Randomised Hadamard transform over the last dim (vq2/vq.py:74-87):
    forward y = blockdiag(H_hb)(sign * x[perm]) * scale, inverse undoes it.
    scale defaults to hb**-0.5."""
    dev = _dev(x, perm, sign, out)
    n = x.shape[-1]
    x2 = _contig(x, "x").reshape(-1, n)
    B = x2.shape[0]
    _perm_sign(perm, sign, n)
    sc = float(hb) ** -0.5 if scale is None else float(scale)
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=dev)
    _contig(out, "out")
    _lib.call("vq2_rht", _p(x2), _dt(x2, "x"), n, _p(out), _dt(out, "out"), n, _p(perm), _p(sign),
              n, int(hb), B, sc, 1 if inverse else 0, _stream(dev))
    return out


def vq_swiglu_rht(gu, inter, perm=None, sign=None, hb=None, scale=None, *, out=None, out_dtype=torch.float32):
    """act = silu(gu[..., :inter]) * gu[..., inter:2*inter], then the forward
    RHT of act (vq2/paged_runtime.py:501-504 fused)."""
    dev = _dev(gu, perm, sign, out)
    inter = int(inter)
    g2 = _contig(gu, "gu").reshape(-1, gu.shape[-1])
    if g2.shape[-1] < 2 * inter:
        raise Vq2Error("gu last dim must be >= 2*inter")
    hb = inter if hb is None else int(hb)
    B = g2.shape[0]
    _perm_sign(perm, sign, inter)
    sc = float(hb) ** -0.5 if scale is None else float(scale)
    if out is None:
        out = torch.empty((*gu.shape[:-1], inter), dtype=out_dtype, device=dev)
    _contig(out, "out")
    _lib.call("vq2_swiglu_rht", _p(g2), _dt(g2, "gu"), g2.shape[-1], inter, _p(out), _dt(out, "out"), inter,
              _p(perm), _p(sign), hb, B, sc, _stream(dev))
    return out


# ------------------------------------------------------------ router / top-1
def vq_router_topk(logits, k=8, h=None, shared_gate=None, shared_id=-1, *, ids=None, w=None):
    """Softmax (fp32) -> top-k -> renormalise per token (transformers
    Qwen3_5MoeTopKRouter).  With shared_id >= 0 an extra slot k carries the
    shared expert with weight sigmoid(shared_gate . h).  Returns
    (ids int32 [T, k(+1)], w float32 [T, k(+1)])."""
    dev = _dev(logits, h, shared_gate, ids, w)
    lg = _contig(logits, "logits").reshape(-1, logits.shape[-1])
    T, E = lg.shape
    extra = 1 if shared_id >= 0 else 0
    hid = 0
    if extra:
        if h is None or shared_gate is None:
            raise Vq2Error("shared expert gate needs h and shared_gate")
        hid = _gate_vec(shared_gate, shared_gate.numel()).numel()
        h = _contig(h, "h").reshape(T, hid)
    if ids is None:
        ids = torch.empty((T, k + extra), dtype=torch.int32, device=dev)
    if w is None:
        w = torch.empty((T, k + extra), dtype=torch.float32, device=dev)
    _lib.call("vq2_router_topk", _p(lg), _dt(lg, "logits"), T, E, int(k), _p(h) if extra else None,
              _dt(h, "h") if extra else 0, hid, _p(shared_gate) if extra else None,
              _dt(shared_gate, "gate") if extra else 0, int(shared_id), _p(ids), _p(w), _stream(dev))
    return ids, w


def vq_argmax(v):
    """First-maximum index per row of v [rows, cols] -> (idx int64, val fp32)."""
    dev = _dev(v)
    v2 = _contig(v, "v").reshape(-1, v.shape[-1])
    idx = torch.empty(v2.shape[0], dtype=torch.int64, device=dev)
    val = torch.empty(v2.shape[0], dtype=torch.float32, device=dev)
    _lib.call("vq2_argmax_rows", _p(v2), _dt(v2, "v"), v2.shape[0], v2.shape[1], _p(idx), _p(val), _stream(dev))
    return idx, val


def vq_gemv_argmax(xr, i0, i1, cb0, cb1, scale, out, n, rs=1.0, *, logits_ws=None):
    """LM head + top-1: (idx int64 [B], val fp32 [B]) of the argmax of the VQ
    GEMV logits (PackedLMHead, vq2/runtime.py:136-144, then torch.argmax)."""
    dev = _dev(xr, i0, i1, cb0, cb1, scale)
    n, out = int(n), int(out)
    x2 = _contig(xr, "xr").reshape(-1, n)
    B = x2.shape[0]
    i0, i1, s2 = _planes(i0, i1, cb0, cb1, scale, out, n)
    idx = torch.empty(B, dtype=torch.int64, device=dev)
    val = torch.empty(B, dtype=torch.float32, device=dev)
    if B < 3 or n % 64:
        # fused top-1 (no logits written) where the shape allows, else logits + top-1
        if logits_ws is None:
            logits_ws = torch.empty((B, out), dtype=torch.float32, device=dev)
        _contig(logits_ws, "logits_ws")
        if logits_ws.dtype != torch.float32 or logits_ws.numel() < B * out:
            raise Vq2Error("logits_ws must be float32 with B * out elements")
        _lib.call("vq2_gemv_argmax", _p(x2), _dt(x2, "xr"), B, x2.stride(0) if B > 1 else n, _p(i0), _p(i1), s2,
                  _p(cb0), _p(cb1), _dt(cb0, "cb0"), _p(scale), _dt(scale, "scale"), out, n, float(rs),
                  _p(logits_ws), _p(idx), _p(val), _stream(dev))
        return idx, val
    else:
        # matrix cores (every centroid gathered once per 64 rows), the top-1
        # fused into the split-K reduce: no logits written
        lib = _lib.load()
        for b0 in range(0, B, 64):
            b1 = min(B, b0 + 64)
            xb = x2[b0:b1]
            ws = _workspace(dev, int(lib.vq2_gemm_small_m_argmax_workspace(b1 - b0, out, n)))
            _lib.call("vq2_gemm_small_m_argmax", _p(xb), _dt(xb, "xr"), b1 - b0, x2.stride(0), _p(i0), _p(i1), s2,
                      _p(cb0), _p(cb1), _dt(cb0, "cb0"), _p(scale), _dt(scale, "scale"), out, n, float(rs), _p(ws),
                      ws.numel(), _p(idx[b0:b1]), _p(val[b0:b1]), _stream(dev))
        return idx, val


# --------------------------------------------------------------- debugging
def vq_dequant_rows(i0, i1, cb0, cb1, scale, r0=0, r1=None):
    """Rotated-space fp32 rows [r1-r0, n] (QMat.dequant before rot.inv,
    vq2/vq.py:283-292): (f32(cb0[i0]) [+ f32(cb1[i1])]) * f32(scale[r])."""
    dev = _dev(i0, i1, cb0, cb1, scale)
    i0 = _idx16(i0, "i0")
    out_rows, ng = i0.shape
    r1 = out_rows if r1 is None else int(r1)
    s2 = _lib.S2_NONE
    if i1 is not None:
        s2 = _lib.S2_U8 if i1.dtype == torch.uint8 else _lib.S2_U16
        if s2 == _lib.S2_U16:
            i1 = _idx16(i1, "i1")
        _contig(i1, "i1")
    y = torch.empty((r1 - int(r0), ng * 8), dtype=torch.float32, device=dev)
    _lib.call("vq2_dequant_rows", _p(i0), _p(i1), s2, _p(_contig(cb0, "cb0")),
              _p(cb1.contiguous()) if cb1 is not None else None, _dt(cb0, "cb0"), _p(_contig(scale, "scale")),
              _dt(scale, "scale"), int(r0), r1, ng * 8, _p(y), _stream(dev))
    return y


def vq_decode_idx(idx):
    """int16 plane -> int32 uint16 codes (& 0xFFFF); uint8 -> int32 values
    (vq2/runtime.py:32-35)."""
    dev = _dev(idx)
    is_u8 = 1 if idx.dtype == torch.uint8 else 0
    if not is_u8:
        idx = _idx16(idx, "idx")
    idx = _contig(idx, "idx")
    out = torch.empty(idx.shape, dtype=torch.int32, device=dev)
    _lib.call("vq2_decode_idx", _p(idx), is_u8, idx.numel(), _p(out), _stream(dev))
    return out


def vq_unpack_fixed(buf, bits, n, *, out=None):
    """Fixed-width packed symbols (uint8 stream, bits in {4, 8, 12, 16}) ->
    int16 [n] holding the uint16 codes, on the device (vq2/export.py:56-70
    unpack_fixed, at container load time)."""
    dev = _dev(buf, out)
    if buf.dtype != torch.uint8:
        raise Vq2Error("buf must be a uint8 tensor")
    b = _contig(buf, "buf").reshape(-1)
    n = int(n)
    if out is None:
        out = torch.empty(n, dtype=torch.int16, device=dev)
    elif out.dtype != torch.int16 or out.numel() < n:
        raise Vq2Error("out must be int16 with at least n elements")
    _lib.call("vq2_unpack_fixed", _p(b), b.numel(), int(bits), n, _p(_contig(out, "out")), _stream(dev))
    return out
