"""Residual-VQ compressed splat attributes decoded on the GPU.

Each attribute (scale: 2, rotation: 4, opacity: 1) is stored as per-splat
uint16 indices [P, stages] into float32 codebooks [stages, K, dim]; decode is
bias + the ordered stage sum (((cb0[i0] + cb1[i1]) + cb2[i2]) + cb3[i3]),
followed by the GaussianModel activations (exp, normalise, sigmoid;
scene/gaussian_model.py:26-41).  The reference has no RVQ; this is the
compressed-attribute workload of the benchmark suite.
"""
from __future__ import annotations

import ctypes as ct
from typing import Dict, Optional

import numpy as np
import torch

from . import _lib as L

ACTIVATION = {"scale": 1, "rotation": 2, "opacity": 3}
DIMS = {"scale": 2, "rotation": 4, "opacity": 1}


def rvq_decode(codebooks: torch.Tensor, indices: torch.Tensor, bias=None, activation: int = 0,
               raw_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """codebooks float32 [S, K, dim] (device), indices uint16/int16 [P, S]
    (device, the 16-bit pattern is the index) -> float32 [P, dim]."""
    if codebooks.dtype != torch.float32 or codebooks.dim() != 3:
        raise ValueError("codebooks must be float32 [stages, K, dim]")
    if indices.element_size() != 2 or indices.dim() != 2:
        raise ValueError("indices must be a 16-bit [P, stages] tensor")
    S, K, dim = codebooks.shape
    P = indices.shape[0]
    if indices.shape[1] != S:
        raise ValueError(f"indices have {indices.shape[1]} stages, codebooks {S}")
    cb = codebooks.contiguous()
    if cb.data_ptr() % 16:
        cb = cb.clone()
    idx = indices.contiguous()
    out = torch.empty((P, dim), dtype=torch.float32, device=cb.device)
    bc = None
    if bias is not None:
        b = np.asarray(bias, dtype=np.float32).reshape(-1)
        bc = (ct.c_float * dim)(*[float(v) for v in b])
    L.check(L.lib().nest_rvq_decode(P, S, K, dim, L.ptr(cb), L.ptr(idx), bc, int(activation), L.ptr(out),
                                    L.ptr(raw_out), L.stream_ptr(cb.device)), "nest_rvq_decode")
    return out


class RVQAttributes:
    """Scale / rotation / opacity of P splats in RVQ form."""

    def __init__(self, codebooks: Dict[str, torch.Tensor], indices: Dict[str, torch.Tensor], bias: Dict[str, tuple]):
        self.codebooks = codebooks
        self.indices = indices
        self.bias = bias

    @classmethod
    def from_numpy(cls, cbs: dict, idxs: dict, bias: dict, device) -> "RVQAttributes":
        cb = {a: torch.from_numpy(np.ascontiguousarray(cbs[a])).to(device) for a in cbs}
        ix = {a: torch.from_numpy(np.ascontiguousarray(idxs[a]).view(np.int16)).to(device) for a in idxs}
        return cls(cb, ix, bias)

    def decode(self, raw: bool = False) -> Dict[str, torch.Tensor]:
        """Decodes the three attributes in one launch (nest_rvq_decode_batch)."""
        out, keep = {}, []
        attrs = (L.RvqAttr * 3)()
        for k, a in enumerate(("scale", "rotation", "opacity")):
            cb = self.codebooks[a]
            idx = self.indices[a]
            if cb.dtype != torch.float32 or cb.dim() != 3 or idx.element_size() != 2 or idx.dim() != 2:
                raise ValueError(f"{a}: codebooks must be float32 [S, K, dim], indices 16-bit [P, S]")
            S, K, dim = cb.shape
            if idx.shape[1] != S:
                raise ValueError(f"{a}: indices have {idx.shape[1]} stages, codebooks {S}")
            cb = cb.contiguous()
            if cb.data_ptr() % 16:
                cb = cb.clone()
            idx = idx.contiguous()
            P = idx.shape[0]
            o = torch.empty((P, dim), dtype=torch.float32, device=cb.device)
            r = torch.empty((P, dim), dtype=torch.float32, device=cb.device) if raw else None
            b = self.bias.get(a)
            bc = None
            if b is not None:
                bv = np.asarray(b, dtype=np.float32).reshape(-1)
                bc = (ct.c_float * dim)(*[float(v) for v in bv])
            keep += [cb, idx, bc]
            attrs[k] = L.RvqAttr(ct.sizeof(L.RvqAttr), P, S, K, dim, ACTIVATION[a], L.ptr(cb), L.ptr(idx),
                                 ct.cast(bc, ct.POINTER(ct.c_float)) if bc is not None else None, L.ptr(o), L.ptr(r))
            out[a] = o
            if raw:
                out[a + "_raw"] = r
        dev = self.codebooks["scale"].device
        L.check(L.lib().nest_rvq_decode_batch(3, attrs, L.stream_ptr(dev)), "nest_rvq_decode_batch")
        return out
