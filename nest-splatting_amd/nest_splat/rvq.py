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
        out = {}
        for a in ("scale", "rotation", "opacity"):
            cb = self.codebooks[a]
            r = torch.empty((self.indices[a].shape[0], cb.shape[2]), dtype=torch.float32, device=cb.device) if raw else None
            out[a] = rvq_decode(cb, self.indices[a], self.bias.get(a), ACTIVATION[a], raw_out=r)
            if raw:
                out[a + "_raw"] = r
        return out
