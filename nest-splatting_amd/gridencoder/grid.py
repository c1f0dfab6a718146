"""Drop-in GridEncoder (forward) on libnest_splat.

Same constructor, attributes and forward signature as gridencoder/grid.py:98-165
of the reference: GridEncoder(input_dim=3, num_levels=16, level_dim=2,
per_level_scale=2, base_resolution=16, log2_hashmap_size=19,
desired_resolution=None, gridtype='hash', align_corners=False,
interpolation='linear'); forward(inputs, bound=1) with inputs in [0, 1]
returns [..., num_levels * level_dim]; get_params() returns (embeddings,
offsets, num_levels, per_level_scale, base_resolution, align_corners,
interp_id).  Under autocast with an even level_dim the table is used in
float16 (GE/grid.py:43-44).  Backward (GE/grid.py:67-91) gives the table
gradient and, when the inputs require grad, the input gradient, for D = 3 and
float32 tables; other cases and total-variation gradients raise
NotImplementedError.
"""
from __future__ import annotations

import ctypes as ct

import numpy as np
import torch
import torch.nn as nn

from nest_splat import _lib as L

_gridtype_to_id = {"hash": 0, "tiled": 1}
_interp_to_id = {"linear": 0, "smoothstep": 1}


def grid_encode_forward(inputs: torch.Tensor, embeddings: torch.Tensor, offsets_host: np.ndarray, per_level_scale: float,
                        base_resolution: int, gridtype: int = 0, align_corners: bool = False,
                        interpolation: int = 0) -> torch.Tensor:
    """_grid_encode.forward (GE/grid.py:27-65) without the permute copy:
    returns [B, L * C] directly."""
    inputs = inputs.contiguous()
    if inputs.dtype != torch.float32:
        inputs = inputs.float()
    B, D = inputs.shape
    L_ = int(offsets_host.shape[0]) - 1
    C = int(embeddings.shape[1])
    S = float(np.log2(per_level_scale))
    if embeddings.dtype == torch.float32:
        code = L.DTYPE_F32
    elif embeddings.dtype == torch.float16:
        code = L.DTYPE_F16
    else:
        raise NotImplementedError(f"embeddings dtype {embeddings.dtype} (float32 / float16 supported)")
    emb = embeddings.detach().contiguous()
    if emb.data_ptr() % 16:
        emb = emb.clone()
    out = torch.empty((B, L_ * C), dtype=emb.dtype, device=inputs.device)
    offs = (ct.c_int32 * (L_ + 1))(*[int(v) for v in offsets_host])
    L.check(L.lib().nest_grid_encode(L.ptr(inputs), B, D, L.ptr(emb), int(emb.shape[0]), code, offs, L_, C, S,
                                     int(base_resolution), int(gridtype), int(bool(align_corners)), int(interpolation),
                                     L.ptr(out), L.stream_ptr(inputs.device)), "nest_grid_encode")
    return out


def grid_encode_backward(inputs: torch.Tensor, embeddings: torch.Tensor, offsets_host: np.ndarray,
                         per_level_scale: float, base_resolution: int, grad: torch.Tensor, calc_grad_inputs: bool,
                         gridtype: int = 0, align_corners: bool = False, interpolation: int = 0):
    """_grid_encode.backward (GE/grid.py:67-91): (grad_inputs or None,
    grad_embeddings) for grad [B, L * C]."""
    inputs = inputs.contiguous()
    if inputs.dtype != torch.float32:
        inputs = inputs.float()
    B, D = inputs.shape
    if D != 3:
        raise NotImplementedError(f"GridEncoder backward supports input_dim 3 (got {D})")
    if embeddings.dtype != torch.float32:
        raise NotImplementedError("GridEncoder backward supports float32 embeddings")
    L_ = int(offsets_host.shape[0]) - 1
    C = int(embeddings.shape[1])
    emb = embeddings.detach().contiguous()
    if emb.data_ptr() % 16:
        emb = emb.clone()
    grad = grad.contiguous().float()
    grad_emb = torch.empty_like(emb)
    grad_in = torch.empty((B, 3), dtype=torch.float32, device=inputs.device) if calc_grad_inputs else None
    offs = (ct.c_int32 * (L_ + 1))(*[int(v) for v in offsets_host])
    L.check(L.lib().nest_grid_encode_backward(L.ptr(inputs), B, D, L.ptr(emb), int(emb.shape[0]), L.DTYPE_F32, offs,
                                              L_, C, float(np.log2(per_level_scale)), int(base_resolution),
                                              int(gridtype), int(bool(align_corners)), int(interpolation),
                                              L.ptr(grad), L.ptr(grad_emb), L.ptr(grad_in),
                                              L.stream_ptr(inputs.device)), "nest_grid_encode_backward")
    return grad_in, grad_emb


class _GridEncode(torch.autograd.Function):
    @staticmethod
    def forward(ctx, inputs, embeddings, offsets_host, per_level_scale, base_resolution, calc_grad_inputs, gridtype,
                align_corners, interpolation):
        if torch.is_autocast_enabled() and embeddings.shape[1] % 2 == 0:
            embeddings = embeddings.to(torch.half)
        ctx.save_for_backward(inputs, embeddings)
        ctx.params = (offsets_host, per_level_scale, base_resolution, bool(calc_grad_inputs), gridtype,
                      align_corners, interpolation)
        return grid_encode_forward(inputs, embeddings, offsets_host, per_level_scale, base_resolution, gridtype,
                                   align_corners, interpolation)

    @staticmethod
    def backward(ctx, grad):
        inputs, embeddings = ctx.saved_tensors
        offsets_host, pls, base, calc, gridtype, align, interp = ctx.params
        grad_in, grad_emb = grid_encode_backward(inputs, embeddings, offsets_host, pls, base, grad, calc, gridtype,
                                                 align, interp)
        if grad_in is not None:
            grad_in = grad_in.to(inputs.dtype)
        return grad_in, grad_emb, None, None, None, None, None, None, None


def grid_encode(inputs, embeddings, offsets, per_level_scale, base_resolution, calc_grad_inputs=False, gridtype=0,
                align_corners=False, interpolation=0):
    """grid_encode = _grid_encode.apply of GE/grid.py:95 (offsets may be a
    device tensor; its host copy is read once)."""
    from nest_splat.rasterizer import host_array
    offsets_host = host_array(offsets, np.int64).astype(np.int64)
    return _GridEncode.apply(inputs, embeddings, offsets_host, per_level_scale, base_resolution, calc_grad_inputs,
                             gridtype, align_corners, interpolation)


class GridEncoder(nn.Module):
    def __init__(self, input_dim=3, num_levels=16, level_dim=2, per_level_scale=2, base_resolution=16,
                 log2_hashmap_size=19, desired_resolution=None, gridtype='hash', align_corners=False,
                 interpolation='linear'):
        super().__init__()
        if desired_resolution is not None:
            per_level_scale = np.exp2(np.log2(desired_resolution / base_resolution) / (num_levels - 1))
        self.input_dim = input_dim
        self.num_levels = num_levels
        self.level_dim = level_dim
        self.per_level_scale = per_level_scale
        self.log2_hashmap_size = log2_hashmap_size
        self.base_resolution = base_resolution
        self.output_dim = num_levels * level_dim
        self.gridtype = gridtype
        self.gridtype_id = _gridtype_to_id[gridtype]
        self.interpolation = interpolation
        self.interp_id = _interp_to_id[interpolation]
        self.align_corners = align_corners
        # uniform per-level table size 2^log2_hashmap_size (GE/grid.py:120-130)
        offsets = [i * (2 ** log2_hashmap_size) for i in range(num_levels + 1)]
        self._offsets_host = np.asarray(offsets, dtype=np.int32)
        self.register_buffer("offsets", torch.from_numpy(self._offsets_host.copy()))
        self.max_params = 2 ** log2_hashmap_size
        self.n_params = offsets[-1] * level_dim
        self.embeddings = nn.Parameter(torch.empty(offsets[-1], level_dim))
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.embeddings)

    def __repr__(self):
        return (f"GridEncoder: input_dim={self.input_dim} num_levels={self.num_levels} level_dim={self.level_dim} "
                f"resolution={self.base_resolution} -> "
                f"{int(round(self.base_resolution * self.per_level_scale ** (self.num_levels - 1)))} "
                f"per_level_scale={self.per_level_scale:.4f} params={tuple(self.embeddings.shape)} "
                f"gridtype={self.gridtype} align_corners={self.align_corners} interpolation={self.interpolation}")

    def forward(self, inputs, bound=1):
        prefix_shape = list(inputs.shape[:-1])
        inputs = inputs.reshape(-1, self.input_dim)
        outputs = _GridEncode.apply(inputs, self.embeddings, self._offsets_host, self.per_level_scale,
                                    self.base_resolution, inputs.requires_grad, self.gridtype_id, self.align_corners,
                                    self.interp_id)
        return outputs.view(prefix_shape + [self.output_dim])

    def get_params(self):
        return self.embeddings, self.offsets, self.num_levels, self.per_level_scale, self.base_resolution, \
            self.align_corners, self.interp_id

    def grad_total_variation(self, weight=1e-7, inputs=None, bound=1, B=1000000):
        raise NotImplementedError("total-variation gradients are a training feature and are not implemented")
