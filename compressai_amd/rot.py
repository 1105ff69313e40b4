"""Incoherence rotation of the VQ2 decode path, run by the HIP RHT kernel.

Mirrors the reference's rotation objects (vq2/vq.py:15-103 and
vq2/runtime.py:37-66):

* ``tag_seed(tag)`` = int(md5(tag)[:8], 16)                    (vq.py:40-41)
* ``Rot(n, seed, device)``: perm = randperm(n), sign = 2*randint(0, 2)-1
  drawn in that order from ``torch.Generator().manual_seed(seed)``; the block
  size hb = min(2048, n) if it is a power of two dividing n, else 2048
  (vq.py:47-56).  ``fwd(x) = blockdiag_hb(H)(sign * x[perm]) * hb**-0.5`` and
  ``inv`` its inverse (vq.py:74-87), computed by ``vq2_rht`` on the GPU.
* ``get_rot(tag, n, device)``: cached ``Rot`` per (tag, n, device) (vq.py:99-103).
* ``FastRot``: the unnormalised transform (scale 1, the 2048**-0.5 deferred to
  the GEMV's ``rs = RS``) cached by input identity and version
  (runtime.py:37-66).

The reference's CUDA bf16 fast path multiplies by a precomputed bf16 matrix
(``x @ M``, vq.py:59-64, 78-82); here the transform is an exact-structure FWHT
in fp32 with a single rounding to the output dtype.
"""
from __future__ import annotations

import hashlib

import torch

from .kernels import vq_rht, Vq2Error

D = 8
HB = 2048


def hadamard(n: int) -> torch.Tensor:
    """Sylvester Hadamard matrix H_n (fp32, CPU), H_{2m} = [[H, H], [H, -H]]."""
    if n <= 0 or n & (n - 1):
        raise ValueError(f"hadamard: n={n} must be a power of two")
    H = torch.ones(1, 1)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H


def tag_seed(tag: str) -> int:
    return int(hashlib.md5(tag.encode()).hexdigest()[:8], 16)


def block_size(n: int) -> int:
    m = min(HB, n)
    return m if (n % m == 0 and (m & (m - 1)) == 0) else HB


def rot_tables(n: int, seed: int):
    """(perm int64 [n], sign float32 [n]) drawn exactly as Rot draws them."""
    g = torch.Generator().manual_seed(int(seed))
    perm = torch.randperm(n, generator=g)
    sign = torch.randint(0, 2, (n,), generator=g).float() * 2 - 1
    return perm, sign


class Rot:
    """x' = R^T x on the last dim (see module docstring)."""

    def __init__(self, n: int, seed: int, device="cuda", perm=None, sign=None):
        self.hb = block_size(n)
        if n % self.hb:
            raise ValueError(f"n={n} is not a multiple of hb={self.hb}")
        self.n, self.nb = n, n // self.hb
        if perm is None or sign is None:
            perm, sign = rot_tables(n, seed)
        self.perm = torch.as_tensor(perm, dtype=torch.int64).to(device)
        self.inv_perm = torch.argsort(self.perm)
        self.sign = torch.as_tensor(sign, dtype=torch.float32).to(device=device, dtype=torch.bfloat16)
        self.sign_bf16 = self.sign
        self.scale = self.hb ** -0.5
        self._perm32 = self.perm.to(torch.int32)
        self._sign8 = self.sign.float().to(torch.int8)

    def fwd(self, x: torch.Tensor, out_dtype=None) -> torch.Tensor:
        return vq_rht(x.contiguous(), self._perm32, self._sign8, self.hb, self.scale, out_dtype=out_dtype)

    def inv(self, y: torch.Tensor, out_dtype=None) -> torch.Tensor:
        return vq_rht(y.contiguous(), self._perm32, self._sign8, self.hb, self.scale, inverse=True,
                      out_dtype=out_dtype)


_ROTS: dict = {}


def get_rot(tag: str, n: int, device="cuda") -> Rot:
    k = (tag, n, str(device))
    if k not in _ROTS:
        _ROTS[k] = Rot(n, tag_seed(tag), device)
    return _ROTS[k]


class FastRot:
    """Decode-time rotation without the 2048**-0.5 factor (the GEMV applies
    it through rs = RS), reused while the same input tensor is unchanged."""

    _ALL: dict = {}

    def __init__(self, rot: Rot, device, out_dtype=None):
        if rot.hb != HB:
            raise Vq2Error(f"FastRot needs hb == {HB} (got {rot.hb})")
        self.rot = rot
        self.out_dtype = out_dtype
        self._x, self._ver, self._y = None, -1, None

    @classmethod
    def get(cls, tag, n, device, rot, out_dtype=None):
        k = (tag, n, str(device))
        if k not in cls._ALL:
            cls._ALL[k] = cls(rot, device, out_dtype)
        return cls._ALL[k]

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self._x is x and self._ver == x._version:
            return self._y
        y = vq_rht(x.reshape(-1).contiguous(), self.rot._perm32, self.rot._sign8, HB, 1.0,
                   out_dtype=self.out_dtype)
        self._x, self._ver, self._y = x, x._version, y
        return y


RS = HB ** -0.5
