"""CPU oracle for the VQ2 decode hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed
CPU baseline).  The product package ``compressai_amd`` never imports it; its
HIP path fails loudly when the extension is missing instead of falling back
here.

Two independent restatements of the reference path live here:

* the C scalar oracle ``vq2_oracle.c`` (built into ``liborc_vq2.so`` with
  ``-ffp-contract=off``), wrapped by the ``orc_*`` functions below;
* a numpy fp64 path (``np_*``) built from ``np.take`` + ``einsum`` and
  ``scipy.linalg.hadamard``, used to cross-check the C code.

Reference semantics (paths relative to the reference repository):

* index decode ``int32(i16) & 0xFFFF``: vq2/kernels.py:47,72,140,171,
  vq2/runtime.py:32-35; ``unpack_fixed``: vq2/export.py:56-70
* dequant: vq2/vq.py:283-292 (before ``rot.inv``)
* VQ GEMV: vq2/kernels.py:32-78; grouped: vq2/kernels.py:117-176 and the CPU
  twins vq2/paged_runtime.py:19-41
* RHT: vq2/vq.py:22-27, 44-87
* MoE layer: vq2/paged_runtime.py:491-511 (T == 1 path) composed with the
  Qwen3.5-MoE router / shared expert of transformers 5.15.0
  (models/qwen3_5_moe/modeling_qwen3_5_moe.py, ``Qwen3_5MoeTopKRouter`` and
  ``Qwen3_5MoeSparseMoeBlock.forward``).

Parity status: every function is pinned by a test in tests/test_oracle_*.py
(closed forms, scipy.linalg.hadamard, exhaustive decode, one-hot codebooks,
linearity, fp64 dense matmul).  The router top-k and the shared-expert gate
restate third-party code (transformers) that no reference test pins; they are
checked only against closed-form identities (softmax over the top-k logits).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liborc_vq2.so"

F32, F16, BF16 = 0, 1, 2
S2_NONE, S2_U8, S2_U16 = 0, 1, 2

_lib = None


def build(force: bool = False) -> Path:
    """Compile the C oracle (make -C oracle)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []), check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.orc_f16_to_f32_n.argtypes = [vp, vp, i64]
        L.orc_bf16_to_f32_n.argtypes = [vp, vp, i64]
        L.orc_f32_to_bf16_n.argtypes = [vp, vp, i64]
        L.orc_f32_to_f16_n.argtypes = [vp, vp, i64]
        L.orc_decode_idx16.argtypes = [vp, vp, i64]
        L.orc_unpack_fixed.argtypes = [vp, i64, i32, i64, vp]
        L.orc_unpack_fixed.restype = i64
        L.orc_dequant_rows.argtypes = [vp, vp, i32, vp, vp, i32, vp, i32, i64, i64, i64, vp]
        L.orc_vq_gemv.argtypes = [vp, i32, i64, i64, vp, vp, i32, vp, vp, i32, vp, i32,
                                  i64, i64, f32, vp, vp]
        L.orc_moe_grouped.argtypes = [vp, i32, i64, vp, i32, i64, vp, i64, vp, i32, vp, i32,
                                      i64, i64, f32, vp, vp]
        L.orc_rht.argtypes = [vp, vp, vp, vp, i64, i64, i64, ctypes.c_double, i32]
        L.orc_rht.restype = i32
        L.orc_argmax_rows.argtypes = [vp, i64, i64, vp]
        _lib = L
    return _lib


# ----------------------------------------------------------------- helpers
def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def dt_code(a: np.ndarray, is_bf16: bool = False) -> int:
    """dtype code of an array: float32 -> F32, float16 -> F16, uint16 holding
    bf16 bits (flagged by ``is_bf16``) -> BF16."""
    if is_bf16:
        assert a.dtype == np.uint16
        return BF16
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise TypeError(f"unsupported float dtype {a.dtype}")


class Arr:
    """A float array plus its dtype code; bf16 is carried as uint16 bits."""

    def __init__(self, a: np.ndarray, code: int | None = None):
        self.a = np.ascontiguousarray(a)
        if code is None:
            code = dt_code(self.a)
        self.code = code

    @staticmethod
    def of(x) -> "Arr":
        if isinstance(x, Arr):
            return x
        # torch tensors are accepted so tests can pass what they feed the GPU
        try:
            import torch

            if isinstance(x, torch.Tensor):
                t = x.detach().cpu().contiguous()
                if t.dtype == torch.bfloat16:
                    return Arr(t.view(torch.int16).numpy().view(np.uint16), BF16)
                if t.dtype == torch.float16:
                    return Arr(t.numpy(), F16)
                if t.dtype == torch.float32:
                    return Arr(t.numpy(), F32)
                raise TypeError(f"unsupported tensor dtype {t.dtype}")
        except ImportError:  # pragma: no cover
            pass
        return Arr(np.asarray(x))

    def f32(self) -> np.ndarray:
        """Exact fp32 values of this array."""
        if self.code == F32:
            return self.a.astype(np.float32)
        if self.code == F16:
            return self.a.astype(np.float32)
        return (self.a.astype(np.uint32) << 16).view(np.float32)


def _np_i16(a) -> np.ndarray:
    try:
        import torch

        if isinstance(a, torch.Tensor):
            a = a.detach().cpu().contiguous().numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.ascontiguousarray(a)


# ------------------------------------------------------------ conversions
def f16_to_f32(h_bits: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h_bits, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def bf16_to_f32(b_bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b_bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_f32_n(_p(b), _p(out), b.size)
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), _p(out), x.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


# ------------------------------------------------------------------ decode
def decode_idx16(idx) -> np.ndarray:
    a = _np_i16(idx).astype(np.int16, copy=False)
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, np.int32)
    lib().orc_decode_idx16(_p(a), _p(out), a.size)
    return out


def unpack_fixed(buf: np.ndarray, bits: int, n: int) -> np.ndarray:
    b = np.ascontiguousarray(buf, dtype=np.uint8)
    out = np.empty(n, np.int32)
    r = lib().orc_unpack_fixed(_p(b), b.size, bits, n, _p(out))
    if r < 0:
        raise ValueError(f"unpack_fixed: bad width {bits} or short buffer")
    return out


# ----------------------------------------------------------------- dequant
def _s2(idx1) -> tuple[np.ndarray | None, int]:
    if idx1 is None:
        return None, S2_NONE
    a = _np_i16(idx1)
    if a.dtype == np.uint8:
        return np.ascontiguousarray(a), S2_U8
    return np.ascontiguousarray(a.astype(np.int16, copy=False)), S2_U16


def dequant_rows(idx0, idx1, cb0, cb1, scale, r0: int = 0, r1: int | None = None) -> np.ndarray:
    """[r1-r0, NG*8] fp32 rotated-space rows (vq2/vq.py:283-292)."""
    i0 = np.ascontiguousarray(_np_i16(idx0).astype(np.int16, copy=False))
    out_rows, ng = i0.shape
    r1 = out_rows if r1 is None else r1
    i1, kind = _s2(idx1)
    c0 = Arr.of(cb0)
    c1 = Arr.of(cb1) if cb1 is not None else None
    if c1 is not None and c1.code != c0.code:
        c1 = Arr(c1.f32(), F32)
        c0 = Arr(c0.f32(), F32)
    s = Arr.of(scale)
    out = np.empty((r1 - r0, ng * 8), np.float32)
    lib().orc_dequant_rows(_p(i0), _p(i1), kind, _p(c0.a), _p(c1.a) if c1 else None, c0.code,
                           _p(s.a), s.code, r0, r1, ng, _p(out))
    return out


# -------------------------------------------------------------------- GEMV
def vq_gemv(x, idx0, idx1, cb0, cb1, scale, rs: float = 1.0):
    """Batched VQ GEMV.  x: [n] or [B, n].  Returns (y32, y64) of shape
    [B, OUT] (fp32 accumulation in a fixed order, and fp64 accumulation)."""
    xa = Arr.of(x)
    xs = xa.a if xa.a.ndim == 2 else xa.a.reshape(1, -1)
    xa = Arr(xs, xa.code)
    B, n = xs.shape
    i0 = np.ascontiguousarray(_np_i16(idx0).astype(np.int16, copy=False))
    out_rows, ng = i0.shape
    assert ng * 8 == n, (ng, n)
    i1, kind = _s2(idx1)
    c0 = Arr.of(cb0)
    c1 = Arr.of(cb1) if cb1 is not None else None
    if c1 is not None and c1.code != c0.code:
        c1 = Arr(c1.f32(), F32)
        c0 = Arr(c0.f32(), F32)
    s = Arr.of(scale)
    y32 = np.empty((B, out_rows), np.float32)
    y64 = np.empty((B, out_rows), np.float64)
    lib().orc_vq_gemv(_p(xa.a), xa.code, B, n, _p(i0), _p(i1), kind, _p(c0.a),
                      _p(c1.a) if c1 else None, c0.code, _p(s.a), s.code, out_rows, n,
                      float(rs), _p(y32), _p(y64))
    return y32, y64


def moe_grouped(x, ids, pool, cb, pool_scale, out_rows: int, ng: int, rs: float = 1.0,
                per_pair_x: bool = False):
    """Grouped per-expert GEMV (vq2/kernels.py:117-176).  x: [NG*8] shared
    (gate_up) or [K, NG*8] per pair (down).  Returns (y32, y64) [K, OUT]."""
    xa = Arr.of(x)
    ida = _np_i16(ids)
    ida = np.ascontiguousarray(ida)
    is64 = 1 if ida.dtype == np.int64 else 0
    if not is64:
        ida = ida.astype(np.int32)
    K = ida.size
    pa = np.ascontiguousarray(_np_i16(pool).astype(np.int16, copy=False))
    E = pa.shape[0]
    c = Arr.of(cb)
    s = Arr.of(pool_scale)
    y32 = np.empty((K, out_rows), np.float32)
    y64 = np.empty((K, out_rows), np.float64)
    lib().orc_moe_grouped(_p(xa.a), xa.code, ng * 8 if per_pair_x else 0, _p(ida), is64, K,
                          _p(pa), E, _p(c.a), c.code, _p(s.a), s.code, out_rows, ng, float(rs),
                          _p(y32), _p(y64))
    return y32, y64


# --------------------------------------------------------------------- RHT
def rht(x, perm=None, sign=None, hb: int = 2048, scale: float | None = None,
        inverse: bool = False) -> np.ndarray:
    """fp64 RHT over the last dim (vq2/vq.py:74-87).  scale defaults to
    hb**-0.5 (the reference normalisation)."""
    xa = Arr.of(x)
    xf = xa.f32().astype(np.float64)
    shp = xf.shape
    n = shp[-1]
    x2 = np.ascontiguousarray(xf.reshape(-1, n))
    y = np.empty_like(x2)
    pa = None if perm is None else np.ascontiguousarray(_np_i16(perm).astype(np.int32))
    sa = None if sign is None else np.ascontiguousarray(_np_i16(sign).astype(np.int8))
    sc = hb ** -0.5 if scale is None else scale
    r = lib().orc_rht(_p(x2), _p(y), _p(pa), _p(sa), n, hb, x2.shape[0], float(sc),
                      1 if inverse else 0)
    if r != 0:
        raise ValueError(f"rht: hb={hb} must be a power of two dividing n={n}")
    return y.reshape(shp)


def argmax_rows(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(np.atleast_2d(v), dtype=np.float64)
    out = np.empty(v.shape[0], np.int64)
    lib().orc_argmax_rows(_p(v), v.shape[0], v.shape[1], _p(out))
    return out


# ------------------------------------------------------ numpy fp64 cross-path
def f64(x) -> np.ndarray:
    """Exact fp64 values of a float array/tensor (float64 passes through)."""
    if isinstance(x, np.ndarray) and x.dtype == np.float64:
        return x
    return Arr.of(x).f32().astype(np.float64)


def np_dequant64(idx0, idx1, cb0, cb1, scale) -> np.ndarray:
    """fp64 dequant by np.take (independent of the C code path)."""
    i0 = _np_i16(idx0).astype(np.int16).view(np.uint16).astype(np.int64)
    W = np.take(Arr.of(cb0).f32().astype(np.float64), i0, axis=0)
    if idx1 is not None:
        a1 = _np_i16(idx1)
        i1 = a1.astype(np.int64) if a1.dtype == np.uint8 else a1.astype(np.int16).view(np.uint16).astype(np.int64)
        W = W + np.take(Arr.of(cb1).f32().astype(np.float64), i1, axis=0)
    s = Arr.of(scale).f32().astype(np.float64)
    return W.reshape(W.shape[0], -1) * s[:, None]


def np_gemv64(x, idx0, idx1, cb0, cb1, scale, rs: float = 1.0) -> np.ndarray:
    W = np_dequant64(idx0, idx1, cb0, cb1, scale)
    xf = np.atleast_2d(f64(x))
    return (xf @ W.T) * rs


def np_rht64(x, perm=None, sign=None, hb: int = 2048, scale: float | None = None) -> np.ndarray:
    from scipy.linalg import hadamard

    xf = np.atleast_2d(f64(x))
    n = xf.shape[-1]
    if perm is not None:
        xf = xf[:, np.asarray(_np_i16(perm), dtype=np.int64)]
    if sign is not None:
        xf = xf * np.asarray(_np_i16(sign), dtype=np.float64)[None, :]
    H = hadamard(hb).astype(np.float64)
    y = (xf.reshape(xf.shape[0], n // hb, hb) @ H).reshape(xf.shape[0], n)
    return y * (hb ** -0.5 if scale is None else scale)


# -------------------------------------------------------------- MoE layer
def router_topk(logits: np.ndarray, k: int = 8):
    """Qwen3.5-MoE router on given logits: softmax (fp32) -> top-k ->
    renormalise.  Ties broken toward the lower expert id.  Returns
    (ids int64 [T, k], weights fp64 [T, k]) in descending-weight order."""
    lg = np.atleast_2d(f64(logits))
    order = np.argsort(-lg, axis=-1, kind="stable")[:, :k]
    top = np.take_along_axis(lg, order, axis=-1)
    w = np.exp(top - top[:, :1])
    w = w / w.sum(axis=-1, keepdims=True)
    return order.astype(np.int64), w


def silu(v):
    return v / (1.0 + np.exp(-v))


def moe_layer(h, logits, cb, gu_pool, gu_scale, dn_pool, dn_scale,
              shared_gu_idx, shared_gu_scale, shared_dn_idx, shared_dn_scale, shared_gate,
              perm2048=None, sign2048=None, perm512=None, sign512=None, top_k: int = 8) -> np.ndarray:
    """fp64 oracle of one MoE layer (config 4), per token t:
        ids, w = router(logits[t]);  xr = RHT_2048(h[t])
        for each routed expert e and the shared expert:
            gu = VQ(gate_up_e) xr ;  act = silu(gu[:I]) * gu[I:]
            y_e = VQ(down_e) RHT_I(act)
        out = sum_k w_k y_{e_k} + sigmoid(shared_gate . h[t]) * y_shared
    (vq2/paged_runtime.py:495-510; transformers Qwen3_5MoeSparseMoeBlock)."""
    H = np.atleast_2d(f64(h))
    T, hid = H.shape
    ids, w = router_topk(logits, top_k)
    gu_pool = _np_i16(gu_pool)
    dn_pool = _np_i16(dn_pool)
    gu_s = Arr.of(gu_scale).f32()
    dn_s = Arr.of(dn_scale).f32()
    gate_v = f64(shared_gate).reshape(-1)
    inter = gu_pool.shape[1] // 2
    out = np.zeros((T, dn_pool.shape[1]), np.float64)
    cache = {}

    def weights(e):
        # only the experts the router selects are dequantized (fp64)
        if e not in cache:
            if e == "shared":
                cache[e] = (np_dequant64(shared_gu_idx, None, cb, None, shared_gu_scale),
                            np_dequant64(shared_dn_idx, None, cb, None, shared_dn_scale))
            else:
                cache[e] = (np_dequant64(gu_pool[e], None, cb, None, gu_s[e]),
                            np_dequant64(dn_pool[e], None, cb, None, dn_s[e]))
        return cache[e]

    def expert(e, xr):
        Wgu, Wdn = weights(e)
        g = Wgu @ xr
        act = silu(g[:inter]) * g[inter:]
        act_r = np_rht64(act, perm512, sign512, hb=min(2048, inter))[0]
        return Wdn @ act_r

    for t in range(T):
        xr = np_rht64(H[t], perm2048, sign2048, hb=min(2048, hid))[0]
        for j in range(top_k):
            out[t] += w[t, j] * expert(int(ids[t, j]), xr)
        sg = 1.0 / (1.0 + np.exp(-(gate_v @ H[t])))
        out[t] += sg * expert("shared", xr)
    return out


def moe_experts(h, ids, w, experts, cb, cb8=None, perm_h=None, sign_h=None, perm_i=None,
                sign_i=None) -> np.ndarray:
    """fp64 oracle of the routed-expert sum of PagedMoEExpert.forward
    (vq2/paged_runtime.py:439-568), per token t:
        xr = RHT_H(h[t]);  [g | u] = VQ(gate_up_e) xr
        out[t] = sum_k w[t, k] * VQ(down_e) RHT_I(silu(g) * u),  e = ids[t, k]
    experts(e) -> (gu_idx0, gu_idx1, gu_scale, dn_idx0, dn_idx1, dn_scale):
    idx1 None for a 2 bpw expert; uint8 planes over the stage-2 codebook cb8
    for a promoted 3 bpw expert, whose dequant is cb[i0] + cb8[i1] times the
    row scale (vq2/paged_runtime.py:376-389; the reference multiplies
    rot.inv of that by the unrotated input, which equals the product of the
    rotated-space weights with RHT_H(x) since the RHT is orthogonal)."""
    H = np.atleast_2d(f64(h))
    T, hid = H.shape
    ids = np.asarray(ids).reshape(T, -1)
    w = f64(w).reshape(T, -1)
    cache = {}
    out = None
    for t in range(T):
        xr = np_rht64(H[t], perm_h, sign_h, hb=min(2048, hid))[0]
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            if e not in cache:
                gu0, gu1, gus, dn0, dn1, dns = experts(e)
                cache[e] = (np_dequant64(gu0, gu1, cb, cb8 if gu1 is not None else None, gus),
                            np_dequant64(dn0, dn1, cb, cb8 if dn1 is not None else None, dns))
            Wgu, Wdn = cache[e]
            g = Wgu @ xr
            inter = g.shape[0] // 2
            act = silu(g[:inter]) * g[inter:]
            y = Wdn @ np_rht64(act, perm_i, sign_i, hb=min(2048, inter))[0]
            if out is None:
                out = np.zeros((T, y.shape[0]), np.float64)
            out[t] += w[t, j] * y
    return out


def max_rel_err(y, ref) -> float:
    """max_i |y_i - ref_i| / max_i |ref_i|, in fp64."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))
