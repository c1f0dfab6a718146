"""Drop-in forward rasterizer for 2D Gaussian surfels with an in-loop hash-grid
texture lookup, running on libnest_splat (gfx950 HIP kernels).

Same call surface as submodules/diff-surfel-rasterization/
diff_surfel_rasterization/__init__.py:21-414 of the reference:
GaussianRasterizationSettings (:277-293), HashGridSettings (:295-302),
GaussianRasterizer(raster_settings, hashgrid_settings).forward(...) returning
(color [C,H,W], radii [P], allmap [14,H,W], trans_avg, cover) (:172, :321-396),
markVisible (:310-319) and rasterize_gaussians (:21-66).

Scope: render mode 0 ("baseline") with every kernel_type (0 Gaussian, 1 beta,
2 flex, 3 general), forward and backward: hash-grid features when
HashGridSettings.L > 0; when L == 0, precomputed per-splat colours or RGB
evaluated from SH coefficients (degree <= 3) in preprocess.  Render modes 4
("cat": per-splat features of the coarse levels ahead of a grid of the fine
ones), 12 ("adaptive_cat", blended with the grid by a per-splat weight), 14
("adaptive_zero", the grid scaled by the weight) and 7 ("adaptive_add", every
level blended), forward and backward, with the reference's packed L
(total << 16 | grid levels << 8 | per-splat levels; the backward
differentiates the grid levels within the active count,
CR/backward.cu:576-612).  Forward only (inference flags, or no consistent
backward in the reference): 12 | 0x100, 14 | 0x100 and 13
("adaptive_cat_fast", with or without the inference flag 0x100); 6
("adaptive", half row and half grid); 8, 9 and 10 ("hybrid_SH*", one
3-channel grid level with per-splat SH colours); 2 and 3 ("baseline_double",
"baseline_blend_double", a second grid at the splat centres from
features_diffuse); 1 and 5 (surface potentials).  The backward returns the
reference's gradients (DSRpy:174-275): means3D, the means2D densification
statistic, SH, colours, opacities, scales, rotations, the hash table, shapes,
and the |grad| sum in the ap_level slot; it needs a float32 hash table and at
most 64 channels.  Modes, kernels and options that the reference implements
for other methods (render mode 11, precomputed covariances) raise
NotImplementedError instead of returning zeros.
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np
import torch
import torch.nn as nn

from nest_splat import rasterizer as _rz
from nest_splat import _lib


def cpu_deep_copy_tuple(input_tuple):
    return tuple(item.cpu().clone() if isinstance(item, torch.Tensor) else item for item in input_tuple)


def _empty(t):
    return t is None or (isinstance(t, torch.Tensor) and t.numel() == 0)


def rasterize_gaussians(means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, homotrans,
                        ap_level, features, offsets, gridrange, features_diffuse, offsets_diffuse, gridrange_diffuse,
                        raster_settings, hashgrid_settings, render_mode, shapes, kernel_type):
    return _RasterizeGaussians.apply(means3D, means2D, sh, colors_precomp, opacities, scales, rotations,
                                     cov3Ds_precomp, homotrans, ap_level, features, offsets, gridrange,
                                     features_diffuse, offsets_diffuse, gridrange_diffuse, raster_settings,
                                     hashgrid_settings, render_mode, shapes, kernel_type)


def _channels(hashgrid_settings) -> int:
    sd = getattr(hashgrid_settings, "shape_dims", None)
    if sd is None or (isinstance(sd, torch.Tensor) and sd.numel() != 3) or (not isinstance(sd, torch.Tensor) and len(sd) != 3):
        return 3
    v = _rz.host_array(sd, np.int64)
    return int(v[2])


def _cat_hash_levels(offsets17: np.ndarray) -> int:
    """Grid levels of render_mode 4 (CR/forward.cu:1231-1238): the largest i
    in 1..16 with offsets[i] > offsets[i-1], offsets padded with zeros to 17
    entries (GR:229-233)."""
    hl = 0
    for i in range(1, 17):
        if offsets17[i] > offsets17[i - 1]:
            hl = i
    return hl


def _mixed_grid(hs, render_mode, level, features, offsets, gridrange):
    """HashGridDesc of render modes 4, 7, 12, 13 and 14 from the reference's packed
    level argument: (total << 16) | (grid levels << 8) | per-splat levels
    (GR:224-226, :395-396; CR/forward.cu:744-767, :971-973, :1228); mode 6
    takes the level argument as the grid's level count (CR/forward.cu:1292)."""
    base_mode = render_mode & 0xFF
    if _empty(features) or _empty(offsets) or _empty(gridrange):
        raise ValueError(f"render_mode {render_mode} needs features, offsets and gridrange")
    offs = np.zeros(17, np.int64)
    o = _rz.host_array(offsets, np.int64).reshape(-1)
    offs[:min(17, o.shape[0])] = o[:17]
    hyb = level & 0xFF
    if base_mode == 4:
        levels, total = _cat_hash_levels(offs), 0
    elif base_mode == 6:
        if not 0 < level <= 16:
            raise NotImplementedError(f"render_mode 6 looks up 1 to 16 grid levels (got {level})")
        levels, total, hyb = level, level, 0
    else:
        levels, total = (level >> 8) & 0xFF, (level >> 16) & 0xFF
    table = features.detach().contiguous() if levels > 0 else None
    return _rz.HashGridDesc(levels=levels, level_dim=int(features.shape[1]), log2_scale=float(hs.S),
                            base_resolution=int(hs.H), table=table, offsets=offs,
                            gridrange=_rz.host_array(gridrange, np.float32), align_corners=bool(hs.align_corners),
                            interpolation=int(hs.interpolation), render_mode=int(render_mode), hybrid_levels=hyb,
                            total_levels=total, active_levels=levels if base_mode == 6 else (level >> 8) & 0xFF)


class _RasterizeGaussians(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means3D, means2D, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, homotrans,
                ap_level, features, offsets, gridrange, features_diffuse, offsets_diffuse, gridrange_diffuse,
                raster_settings, hashgrid_settings, render_mode, shapes, kernel_type):
        base_mode = render_mode & 0xFF
        if base_mode not in (0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 13, 14) or (render_mode & ~0x1FF) or \
                ((render_mode & 0x100) and base_mode not in (12, 13, 14)):
            raise NotImplementedError(f"render_mode {render_mode}: implemented are 0 (baseline), 1 / 5 (surface "
                                      f"potentials), 2 / 3 (baseline_double / baseline_blend_double), 4 (cat), "
                                      f"6 (adaptive), 7 (adaptive_add), 8 / 9 / 10 (hybrid_SH / hybrid_SH_post / hybrid_SH_raw) and "
                                      f"12 / 13 / 14 (adaptive_cat / adaptive_cat_fast / adaptive_zero, | 0x100 "
                                      f"inference)")
        if kernel_type not in (0, 1, 2, 3):
            raise NotImplementedError(f"kernel_type {kernel_type}: implemented are 0 (Gaussian), 1 (beta), 2 (flex) "
                                      f"and 3 (general)")
        if kernel_type != 0 and _empty(shapes):
            raise ValueError(f"kernel_type {kernel_type} needs shapes [P] (CR/forward.cu:864-900)")
        if not _empty(cov3Ds_precomp):
            raise NotImplementedError("precomputed transforms (cov3D_precomp) are not implemented")
        if not _empty(features_diffuse) and base_mode not in (1, 2, 3, 5):
            raise NotImplementedError("a second (diffuse) hash grid is read by render modes 1, 2 and 3 only")
        C = _channels(hashgrid_settings)
        level = int(hashgrid_settings.L)
        second_grid = not (_empty(features_diffuse) or _empty(offsets_diffuse) or _empty(gridrange_diffuse))
        if base_mode in (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 14) and level == 0:
            base_mode = render_mode = 0  # level 0 is the colour path in every mode but 13 (CR/forward.cu:1091)
        if base_mode in (1, 2, 3, 5):
            # baseline_double / baseline_blend_double (CR/forward.cu:1146-1217): the grid's
            # levels plus a second grid (features_diffuse, GR's diffuse grid) at the splat
            # centres, 4 features per level in both; surface potentials (1, 5,
            # :1825-1908): 12 or 15 features per level, mode 1 with the second grid
            second = base_mode in (1, 2, 3) and second_grid
            if _empty(features) or _empty(offsets) or _empty(gridrange):
                raise ValueError(f"render_mode {base_mode} needs features, offsets and gridrange")
            hs = hashgrid_settings
            grid = _rz.HashGridDesc(levels=level, level_dim=int(features.shape[1]), log2_scale=float(hs.S),
                                    base_resolution=int(hs.H), table=features.detach().contiguous(),
                                    offsets=_rz.host_array(offsets, np.int64),
                                    gridrange=_rz.host_array(gridrange, np.float32),
                                    align_corners=bool(hs.align_corners), interpolation=int(hs.interpolation),
                                    render_mode=base_mode,
                                    table2=features_diffuse.detach().contiguous() if second else None,
                                    offsets2=_rz.host_array(offsets_diffuse, np.int64) if second else None,
                                    gridrange2=_rz.host_array(gridrange_diffuse, np.float32) if second else None)
            colors = None
        elif base_mode in (8, 9, 10):
            # hybrid SH (CR/forward.cu:1378-1542): level = decompose << 24 | SH degree << 16 |
            # grid levels << 8 (GR:617-626), one 3-channel grid level, rows of 3 raw colours or
            # 48 SH coefficients in colors_precomp
            dec, hl = (level >> 24) & 0xFF, (level >> 8) & 0xFF
            if hl > 1:
                raise NotImplementedError(f"render_mode {base_mode} looks up one grid level (got {hl})")
            if hl and (_empty(features) or _empty(offsets) or _empty(gridrange)):
                raise ValueError(f"render_mode {base_mode} needs features, offsets and gridrange")
            if _empty(colors_precomp):
                raise ValueError(f"render_mode {base_mode} needs the per-splat rows in colors_precomp")
            hs = hashgrid_settings
            grid = _rz.HashGridDesc(levels=hl, level_dim=int(features.shape[1]) if hl else 3,
                                    log2_scale=float(hs.S), base_resolution=int(hs.H),
                                    table=features.detach().contiguous() if hl else None,
                                    offsets=_rz.host_array(offsets, np.int64) if hl else np.zeros(1, np.int64),
                                    gridrange=_rz.host_array(gridrange, np.float32) if hl else
                                    np.zeros(2, np.float32), align_corners=bool(hs.align_corners),
                                    interpolation=int(hs.interpolation), render_mode=base_mode, decompose=dec)
            colors = colors_precomp.detach()
            width = grid.row_width(C)
            if colors.dim() != 2 or colors.shape[1] != width:
                raise ValueError(f"render_mode {base_mode}: colors_precomp must be [P, {width}]")
            level = 1  # no SH colours
        elif base_mode != 0:
            grid = _mixed_grid(hashgrid_settings, render_mode, level, features, offsets, gridrange)
            colors = None if _empty(colors_precomp) else colors_precomp.detach()
            width = grid.row_width(C)
            if colors is not None and (colors.dim() != 2 or colors.shape[1] != width):
                raise ValueError(f"render_mode {render_mode}: colors_precomp must be [P, {width}]")
            level = 1  # no SH colours
        elif level > 0:
            if _empty(features) or _empty(offsets) or _empty(gridrange):
                raise ValueError("hash-grid rendering (L > 0) needs features, offsets and gridrange")
            grid = _rz.HashGridDesc(levels=level, level_dim=int(features.shape[1]),
                                    log2_scale=float(hashgrid_settings.S), base_resolution=int(hashgrid_settings.H),
                                    table=features.detach().contiguous(), offsets=_rz.host_array(offsets, np.int64),
                                    gridrange=_rz.host_array(gridrange, np.float32),
                                    align_corners=bool(hashgrid_settings.align_corners),
                                    interpolation=int(hashgrid_settings.interpolation))
            colors = None
        else:
            grid = _rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
            if _empty(colors_precomp):
                # colours from SH in preprocess (CR/forward.cu:417-424); RGB only
                # (CR/rasterizer_impl.cu:320-323)
                if _empty(sh):
                    raise ValueError("the colour path (L == 0) needs colors_precomp or shs")
                if C != 3:
                    raise RuntimeError("For non-RGB, provide precomputed Gaussian colors!")
                colors = None
            else:
                colors = colors_precomp.detach()
                if colors.dim() != 2 or colors.shape[1] != C:
                    raise ValueError(f"colors_precomp must be [P, {C}] (shape_dims[2])")
        s = raster_settings
        settings = _rz.make_settings(s.image_height, s.image_width, s.tanfovx, s.tanfovy, s.viewmatrix, s.projmatrix,
                                     s.campos, s.scale_modifier, s.beta, s.if_contract, s.max_intersections,
                                     s.prefiltered, s.debug)
        res = _rz.rasterize_forward(settings, grid, means3D.detach(), opacities.detach(), scales.detach(),
                                    rotations.detach(), homotrans=None if _empty(homotrans) else homotrans.detach(),
                                    ap_level=None if _empty(ap_level) else ap_level.detach(), colors_precomp=colors,
                                    channels=C, shs=None if (level > 0 or colors is not None or _empty(sh)) else
                                    sh.detach(), sh_degree=int(raster_settings.sh_degree),
                                    record_transmittance=bool(raster_settings.record_transmittance),
                                    shapes=None if kernel_type == 0 else shapes.detach().reshape(-1),
                                    kernel_type=int(kernel_type))
        ctx.num_rendered = res.num_rendered
        ctx.render_mode = render_mode
        ctx.kernel_type = int(kernel_type)
        ctx.fw = dict(res=res, settings=settings, grid=grid, C=C, colors=colors,
                      shapes=None if kernel_type == 0 else shapes.detach().reshape(-1),
                      shs=None if (level > 0 or colors is not None or _empty(sh)) else sh.detach(),
                      sh_degree=int(raster_settings.sh_degree),
                      homotrans=None if _empty(homotrans) else homotrans.detach(),
                      ap_level=None if _empty(ap_level) else ap_level.detach())
        ctx.save_for_backward(means3D, opacities, scales, rotations)
        ctx.shapes_shape = None if kernel_type == 0 else tuple(shapes.shape)
        dev = means3D.device
        if res.trans_avg is not None:
            # [P, 1] each, as DSR/rasterize_points.cu:169-171 allocates them
            trans_avg, cover = res.trans_avg.view(-1, 1), res.cover_pixels.view(-1, 1)
        else:
            trans_avg = torch.zeros((0, 1), dtype=torch.float32, device=dev)
            cover = torch.zeros((0, 1), dtype=torch.float32, device=dev)
        ctx.mark_non_differentiable(trans_avg, cover)
        return res.color, res.radii, res.others, trans_avg, cover

    @staticmethod
    def backward(ctx, grad_out_color, grad_radii, grad_depth, grad_0, grad_1):
        if ctx.render_mode not in (0, 4, 7, 12, 14):
            raise NotImplementedError(f"render_mode {ctx.render_mode} is forward-only here; "
                                      f"the backward covers modes 0, 4, 7, 12 and 14 (training)")
        means3D, opacities, scales, rotations = ctx.saved_tensors
        fw = ctx.fw
        g = _rz.rasterize_backward(fw["settings"], fw["grid"], fw["res"], means3D.detach(), opacities.detach(),
                                   scales.detach(), rotations.detach(), grad_out_color, grad_depth,
                                   homotrans=fw["homotrans"], ap_level=fw["ap_level"], colors_precomp=fw["colors"],
                                   channels=fw["C"], shs=fw["shs"], sh_degree=fw["sh_degree"], shapes=fw["shapes"],
                                   kernel_type=ctx.kernel_type)
        need = ctx.needs_input_grad

        def pick(i, t, shape=None):
            if not need[i] or t is None:
                return None
            return t.reshape(shape) if shape is not None else t

        ap = fw["ap_level"]
        return (pick(0, g.dmeans3D), pick(1, g.dmeans2D), pick(2, g.dshs), pick(3, g.dcolors),
                pick(4, g.dopacity, opacities.shape), pick(5, g.dscales), pick(6, g.drotations), None, None,
                pick(9, g.dgradsum, None if ap is None else ap.shape), pick(10, g.dfeatures),
                None, None, None, None, None, None, None, None, pick(19, g.dshapes, ctx.shapes_shape), None)


class GaussianRasterizationSettings(NamedTuple):
    image_height: int
    image_width: int
    tanfovx: float
    tanfovy: float
    bg: torch.Tensor
    scale_modifier: float
    viewmatrix: torch.Tensor
    projmatrix: torch.Tensor
    sh_degree: int
    campos: torch.Tensor
    prefiltered: bool
    debug: bool
    beta: float
    if_contract: bool
    record_transmittance: bool
    max_intersections: int = 0  # 0 means no limit


class HashGridSettings(NamedTuple):
    L: int
    S: float
    H: int
    align_corners: bool
    interpolation: int
    shape_dims: torch.Tensor  # [GS, HS, OS]


class GaussianRasterizer(nn.Module):
    def __init__(self, raster_settings, hashgrid_settings):
        super().__init__()
        self.raster_settings = raster_settings
        self.hashgrid_settings = hashgrid_settings

    def markVisible(self, positions):
        # Mark visible points (based on frustum culling for camera) with a boolean
        with torch.no_grad():
            return _rz.mark_visible(positions, self.raster_settings.viewmatrix)

    def forward(self, means3D, means2D, opacities, shs=None, colors_precomp=None, scales=None, rotations=None,
                cov3D_precomp=None, homotrans=None, ap_level=None, features=None, offsets=None, gridrange=None,
                features_diffuse=None, offsets_diffuse=None, gridrange_diffuse=None, render_mode=0, shapes=None,
                kernel_type=0):
        if (shs is None and colors_precomp is None) or (shs is not None and colors_precomp is not None):
            raise Exception('Please provide excatly one of either SHs or precomputed colors!')
        if ((scales is None or rotations is None) and cov3D_precomp is None) or \
                ((scales is not None or rotations is not None) and cov3D_precomp is not None):
            raise Exception('Please provide exactly one of either scale/rotation pair or precomputed 3D covariance!')
        return rasterize_gaussians(means3D, means2D, shs, colors_precomp, opacities, scales, rotations, cov3D_precomp,
                                   homotrans, ap_level, features, offsets, gridrange, features_diffuse,
                                   offsets_diffuse, gridrange_diffuse, self.raster_settings, self.hashgrid_settings,
                                   render_mode, shapes, kernel_type)


def compute_relocation(opacity_old, scale_old, N, binoms, n_max):
    raise NotImplementedError("MCMC relocation belongs to training and is not part of this forward renderer")
