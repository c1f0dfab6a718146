"""render(): counterpart of the baseline hash-textured branch of
gaussian_renderer/__init__.py:23-1062 (parameter gathering :178-213, raster
settings and call :694-760, allmap post-processing :762-797, MLP decode, mask
and background :905-1021, output keys :1025-1046).

The rasterizer runs through the drop-in diff_surfel_rasterization API; the MLP
decode runs fused (view directions, SH encoding, MLP, sigmoid, mask,
background) in one kernel on the channel-major feature map, so the
permute().contiguous() copy of the reference disappears.

The SH-rasterised appearance modes (gaussian_renderer/__init__.py:88-114,
:686-692, :799-903) compose the same kernels: ``diffuse`` and ``specular``
rasterise SH colours (degree 0, resp. the active degree); ``diffuse_ngp`` adds
the hash grid's MLP colour at the back-projected median depth; and
``diffuse_offset`` queries the grid at that point moved by the rendered
colour - 0.5 (clamped to +-0.1), or at the blended splat centres of allmap
8:11 with ``use_xyz_mode``.  The hybrid SH modes (:600-680, :958-1000) pass
raw SH colours or the SH coefficients to render modes 8-10 with a one-level
3-channel grid.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as torch_F

from . import rasterizer as rz
from .camera import Camera, view_ray_matrix
from .mlp import NestMLP


def build_rotation(r: torch.Tensor) -> torch.Tensor:
    """utils/general_utils.py:78-99."""
    norm = torch.sqrt(r[:, 0] * r[:, 0] + r[:, 1] * r[:, 1] + r[:, 2] * r[:, 2] + r[:, 3] * r[:, 3])
    q = r / norm[:, None]
    R = torch.zeros((q.size(0), 3, 3), device=r.device)
    w, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    R[:, 0, 0] = 1 - 2 * (y * y + z * z)
    R[:, 0, 1] = 2 * (x * y - w * z)
    R[:, 0, 2] = 2 * (x * z + w * y)
    R[:, 1, 0] = 2 * (x * y + w * z)
    R[:, 1, 1] = 1 - 2 * (x * x + z * z)
    R[:, 1, 2] = 2 * (y * z - w * x)
    R[:, 2, 0] = 2 * (x * z - w * y)
    R[:, 2, 1] = 2 * (y * z + w * x)
    R[:, 2, 2] = 1 - 2 * (x * x + y * y)
    return R


def build_H(rots: torch.Tensor, scales: torch.Tensor, xyzs: torch.Tensor) -> torch.Tensor:
    """utils/general_utils.py:101-113."""
    batch = rots.shape[0]
    s = torch.zeros(batch, 1, 3, device=rots.device)
    s[:, 0, :2] = scales
    h = torch.zeros(batch, 4, 4, device=rots.device)
    h[:, :3, :3] = torch.mul(s, rots)
    h[:, :3, 3] = xyzs
    h[:, 3, 3] = 1.0
    return h


class SplatModel:
    """The GaussianModel getters the forward render reads
    (scene/gaussian_model.py:231-317), over activated attributes."""

    def __init__(self, xyz, scaling, rotation, opacity, ap_level=None, homotrans=None, features=None,
                 active_sh_degree: int = 0):
        self._xyz = xyz
        self._scaling = scaling
        self._rotation = rotation
        self._opacity = opacity.reshape(-1, 1)
        self._ap = ap_level if ap_level is not None else torch.full((xyz.shape[0], 1), 24.0, device=xyz.device)
        self._homotrans = homotrans
        self._features = features  # [P, (max_sh_degree + 1)^2, 3] SH coefficients, DC first
        self.active_sh_degree = active_sh_degree

    @property
    def get_features(self):
        return self._features

    @property
    def get_xyz(self):
        return self._xyz

    @property
    def get_scaling(self):
        return self._scaling

    @property
    def get_rotation(self):
        return self._rotation

    @property
    def get_opacity(self):
        return self._opacity

    @property
    def get_appearance_level(self):
        return self._ap

    def get_homotrans(self):
        if self._homotrans is not None:
            return self._homotrans
        if self._rotation.is_cuda:
            from .rasterizer import build_homotrans
            return build_homotrans(self._rotation, self._scaling, self._xyz)
        return build_H(build_rotation(self._rotation), self._scaling, self._xyz)


class HashINGP:
    """The INGP attributes the baseline render reads (hash_encoder/modules.py):
    hash_encoding (a GridEncoder), gridrange, contract, active_levels, levels,
    level_dim and rgb_decode."""

    def __init__(self, encoding, mlp: NestMLP, gridrange, contract: bool = False, active_levels: Optional[int] = None):
        self.hash_encoding = encoding
        self.mlp_rgb = mlp
        self.gridrange = torch.as_tensor(np.asarray(gridrange, dtype=np.float32))
        self._gridrange_host = np.asarray(gridrange, dtype=np.float32)
        self.contract = contract
        self.levels = encoding.num_levels
        self.level_dim = encoding.level_dim
        self.active_levels = self.levels if active_levels is None else active_levels

    def rgb_decode(self, features, ray_unit):
        return self.mlp_rgb.rgb_decode(features, ray_unit)

    def __call__(self, points_3D: torch.Tensor, with_xyz: bool = False) -> torch.Tensor:
        """INGP.forward (hash_encoder/modules.py:574-585): grid features of
        world points [N, 3], the levels past active_levels masked to zero."""
        feat = self.encode_3D(points_3D)
        if self.active_levels < self.levels:
            mask = torch.zeros_like(feat)
            mask[..., :self.active_levels * self.level_dim] = 1
            feat = feat * mask
        if with_xyz:
            feat = torch.cat([feat, points_3D], dim=-1)
        return feat.float()

    def encode_3D(self, points_3D: torch.Tensor) -> torch.Tensor:
        """INGP._encode_3D (hash_encoder/modules.py:697-725): normalise to
        [0, 1] over the grid range (through the contraction of the space
        outside the unit ball when contract is set), then the GridEncoder."""
        vol_min, vol_max = float(self._gridrange_host[0]), float(self._gridrange_host[1])
        if not self.contract:
            x = (points_3D - vol_min) / (vol_max - vol_min)
        else:
            vmid = (vol_min + vol_max) * 0.5
            vsize = (vol_max - vol_min) * 0.5
            x = (points_3D - vmid) / vsize
            norm = x.norm(dim=-1, keepdim=True)
            inv_norm = 1.0 / norm
            x = x * torch.where(norm <= 1.0, torch.ones_like(norm), (2.0 - inv_norm) * inv_norm)
            x = (x + 2.0) * 0.25
        out = self.hash_encoding(x.reshape(-1, 3))
        return out.view(*x.shape[:-1], out.shape[-1])


@dataclass
class Pipe:
    depth_ratio: float = 0.0


def _matrix(x, device) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=torch.float32)
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(device)


def cam2rays(cam, device) -> tuple:
    """utils/point_utils.py:31-46: per-pixel ray directions [H*W, 3] (row
    major, not normalised) and the camera centre [3]."""
    W, H = cam.image_width, cam.image_height
    wv = _matrix(cam.world_view_transform, device)
    c2w = torch.linalg.inv(wv.T)
    M = torch.from_numpy(view_ray_matrix(cam)).to(device)
    gx, gy = torch.meshgrid(torch.arange(W, device=device).float(), torch.arange(H, device=device).float(),
                            indexing="xy")
    pts = torch.stack([gx, gy, torch.ones_like(gx)], dim=-1).reshape(-1, 3)
    return pts @ M, c2w[:3, 3]


def depths_to_points(cam, depth: torch.Tensor) -> tuple:
    """utils/point_utils.py:10-29: the depth map [1, H, W] back-projected
    along the pixel rays; returns points [H*W, 3], rays_d, rays_o."""
    rays_d, rays_o = cam2rays(cam, depth.device)
    return depth.reshape(-1, 1) * rays_d + rays_o, rays_d, rays_o


def depth_to_normal(cam, depth: torch.Tensor) -> torch.Tensor:
    """utils/point_utils.py:48-60."""
    W, H = cam.image_width, cam.image_height
    points = depths_to_points(cam, depth)[0].reshape(H, W, 3)
    out = torch.zeros_like(points)
    dx = points[2:, 1:-1] - points[:-2, 1:-1]
    dy = points[1:-1, 2:] - points[1:-1, :-2]
    out[1:-1, 1:-1, :] = torch_F.normalize(torch.cross(dx, dy, dim=-1), dim=-1)
    return out


SH_MODES = ("diffuse", "specular", "diffuse_ngp", "diffuse_offset")
# the reference's hybrid SH methods and their render_mode (GR:600-680)
HYBRID_MODES = {"hybrid_SH": 8, "hybrid_SH_post": 9, "hybrid_SH_raw": 10}
DECOMPOSE = {None: 0, "gaussian_only": 1, "ngp_only": 2}

# Real spherical-harmonic basis constants up to degree 3 (the normalisation
# of the real SH Y_lm; the same values as the preprocess kernel's).
_SH_C0 = 0.28209479177387814
_SH_C1 = 0.4886025119029199
_SH_C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792, 0.5462742152960396)
_SH_C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154, -0.4570457994644658,
          1.445305721320277, -0.5900435899266435)


def eval_sh(deg: int, sh: torch.Tensor, dirs: torch.Tensor) -> torch.Tensor:
    """utils/sh_utils.py:57-117: SH coefficients sh [..., C, (deg+1)^2 or
    more] at unit directions dirs [..., 3] -> [..., C], no activation."""
    x, y, z = dirs[..., 0:1], dirs[..., 1:2], dirs[..., 2:3]
    r = _SH_C0 * sh[..., 0]
    if deg > 0:
        r = r - _SH_C1 * y * sh[..., 1] + _SH_C1 * z * sh[..., 2] - _SH_C1 * x * sh[..., 3]
        if deg > 1:
            xx, yy, zz = x * x, y * y, z * z
            xy, yz, xz = x * y, y * z, x * z
            r = (r + _SH_C2[0] * xy * sh[..., 4] + _SH_C2[1] * yz * sh[..., 5] +
                 _SH_C2[2] * (2.0 * zz - xx - yy) * sh[..., 6] + _SH_C2[3] * xz * sh[..., 7] +
                 _SH_C2[4] * (xx - yy) * sh[..., 8])
            if deg > 2:
                r = (r + _SH_C3[0] * y * (3 * xx - yy) * sh[..., 9] + _SH_C3[1] * xy * z * sh[..., 10] +
                     _SH_C3[2] * y * (4 * zz - xx - yy) * sh[..., 11] +
                     _SH_C3[3] * z * (2 * zz - 3 * xx - 3 * yy) * sh[..., 12] +
                     _SH_C3[4] * x * (4 * zz - xx - yy) * sh[..., 13] + _SH_C3[5] * z * (xx - yy) * sh[..., 14] +
                     _SH_C3[6] * x * (xx - 3 * yy) * sh[..., 15])
    return r


def render(viewpoint_camera, pc, pipe, bg_color: torch.Tensor, scaling_modifier=1.0, ingp: HashINGP = None, beta=0,
           max_intersections=0, skip_mlp=False, with_surface=True, mode: str = "baseline", use_xyz_mode: bool = False,
           record_transmittance: bool = False, decompose_mode: Optional[str] = None):
    """mode: "baseline" (the hash grid rasterised in the kernel, then the MLP),
    one of the SH-rasterised modes "diffuse", "specular", "diffuse_ngp",
    "diffuse_offset", or one of the hybrid SH modes "hybrid_SH",
    "hybrid_SH_raw", "hybrid_SH_post" with decompose_mode None,
    "gaussian_only" or "ngp_only" (the reference's ingp.is_*_mode flags)."""
    if mode in SH_MODES:
        return _render_sh(viewpoint_camera, pc, pipe, bg_color, scaling_modifier, ingp, beta, max_intersections,
                          with_surface, mode, use_xyz_mode, record_transmittance)
    if mode in HYBRID_MODES:
        return _render_hybrid(viewpoint_camera, pc, pipe, bg_color, scaling_modifier, ingp, beta, max_intersections,
                              with_surface, mode, decompose_mode, record_transmittance)
    if mode != "baseline":
        raise ValueError(f"mode must be 'baseline' or one of {SH_MODES + tuple(HYBRID_MODES)} (got {mode!r})")
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings

    dev = pc.get_xyz.device
    tanfovx = math.tan(viewpoint_camera.FoVx * 0.5)
    tanfovy = math.tan(viewpoint_camera.FoVy * 0.5)
    means3D = pc.get_xyz
    means2D = torch.zeros_like(means3D)
    enc = ingp.hash_encoding
    features, offsets, _, per_level_scale, base_resolution, align_corners, interpolation = enc.get_params()
    host = getattr(enc, "_offsets_host", None)
    if host is not None:
        offsets._nest_host_copy = (offsets._version, np.asarray(host, dtype=np.float64).astype(np.int64))
    gridrange = ingp.gridrange
    gridrange._nest_host_copy = (gridrange._version, ingp._gridrange_host)
    levels = ingp.active_levels
    output_dim = ingp.levels * ingp.level_dim
    shape_dims = torch.tensor([0, output_dim, output_dim], dtype=torch.int32)
    raster_settings = GaussianRasterizationSettings(
        image_height=int(viewpoint_camera.image_height), image_width=int(viewpoint_camera.image_width),
        tanfovx=tanfovx, tanfovy=tanfovy, bg=bg_color, scale_modifier=scaling_modifier,
        viewmatrix=viewpoint_camera.world_view_transform, projmatrix=viewpoint_camera.full_proj_transform,
        sh_degree=0, campos=viewpoint_camera.camera_center, prefiltered=False, debug=False, beta=beta,
        if_contract=ingp.contract, record_transmittance=False, max_intersections=max_intersections)
    hashgrid_settings = HashGridSettings(L=levels, S=math.log2(per_level_scale), H=base_resolution,
                                         align_corners=align_corners, interpolation=interpolation,
                                         shape_dims=shape_dims)
    rasterizer = GaussianRasterizer(raster_settings=raster_settings, hashgrid_settings=hashgrid_settings)
    shs = torch.empty((0,), device=dev)
    rendered_image, radii, allmap, _, _ = rasterizer(
        means3D=means3D, means2D=means2D, shs=shs, colors_precomp=None, opacities=pc.get_opacity,
        scales=pc.get_scaling, rotations=pc.get_rotation, homotrans=pc.get_homotrans(),
        ap_level=pc.get_appearance_level, cov3D_precomp=None, features=features, offsets=offsets,
        gridrange=gridrange, render_mode=0, shapes=None, kernel_type=0)

    render_alpha = allmap[1:2]
    rets = {"viewspace_points": means2D, "visibility_filter": radii > 0, "radii": radii, "features": rendered_image,
            "allmap": allmap}
    H, W = int(viewpoint_camera.image_height), int(viewpoint_camera.image_width)
    if skip_mlp:
        rgb = torch.zeros(3, H, W, device=dev)
        if bg_color.sum() > 0:
            rgb = rgb + (1.0 - render_alpha) * bg_color.to(dev).unsqueeze(-1).unsqueeze(-1)
    else:
        bg = bg_color if float(bg_color.sum()) > 0 else None
        rgb = ingp.mlp_rgb.decode_image(rendered_image, view_ray_matrix(viewpoint_camera), alpha=render_alpha, bg=bg)
    rets["render"] = rgb

    if with_surface:
        rets.update(surface_maps(viewpoint_camera, allmap, getattr(pipe, "depth_ratio", 0.0)))
    return rets


def _render_sh(cam, pc, pipe, bg_color, scaling_modifier, ingp, beta, max_intersections, with_surface, mode,
               use_xyz_mode, record_transmittance):
    """gaussian_renderer/__init__.py:88-114 (mode flags, no grid in the
    rasteriser), :686-760 (SH degree 0 for the diffuse modes), :799-903 (the
    grid queried at the back-projected median depth, or offset by the rendered
    colour), :1013-1046 (background and output keys)."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings

    if pc.get_features is None:
        raise ValueError(f"mode {mode!r} rasterises SH colours: the splat model needs features")
    if mode in ("diffuse_ngp", "diffuse_offset") and ingp is None:
        raise ValueError(f"mode {mode!r} queries the hash grid: pass ingp")
    dev = pc.get_xyz.device
    H, W = int(cam.image_height), int(cam.image_width)
    means2D = torch.zeros_like(pc.get_xyz)
    raster_settings = GaussianRasterizationSettings(
        image_height=H, image_width=W, tanfovx=math.tan(cam.FoVx * 0.5), tanfovy=math.tan(cam.FoVy * 0.5),
        bg=bg_color, scale_modifier=scaling_modifier, viewmatrix=cam.world_view_transform,
        projmatrix=cam.full_proj_transform, sh_degree=0 if mode != "specular" else int(pc.active_sh_degree),
        campos=cam.camera_center, prefiltered=False, debug=False, beta=beta, if_contract=False,
        record_transmittance=record_transmittance, max_intersections=max_intersections)
    hashgrid_settings = HashGridSettings(L=0, S=0.0, H=0, align_corners=False, interpolation=0,
                                         shape_dims=torch.tensor([0, 3, 3], dtype=torch.int32))
    rasterizer = GaussianRasterizer(raster_settings=raster_settings, hashgrid_settings=hashgrid_settings)
    image, radii, allmap, trans_avg, cover = rasterizer(
        means3D=pc.get_xyz, means2D=means2D, shs=pc.get_features, colors_precomp=None, opacities=pc.get_opacity,
        scales=pc.get_scaling, rotations=pc.get_rotation)
    render_alpha = allmap[1:2]
    rets = {"viewspace_points": means2D, "visibility_filter": radii > 0, "radii": radii, "allmap": allmap}
    if mode in ("diffuse_ngp", "diffuse_offset"):
        mask = render_alpha > 0
        median = torch.nan_to_num(allmap[5:6], 0, 0)
        if mode == "diffuse_ngp":
            rets["gaussian_rgb"] = image.clone()
            points, rays_d, _ = depths_to_points(cam, median.detach())
        else:
            # the rendered colour minus 0.5 is the offset, clamped to +-0.1
            offset = torch.clamp(image.permute(1, 2, 0).reshape(-1, 3) - 0.5, -0.1, 0.1)
            rets["gaussian_rgb"] = image.clone() - 0.5
            if use_xyz_mode:
                base = allmap[8:11].permute(1, 2, 0).reshape(-1, 3)
                points = base.detach() + offset
                rays_d, _ = cam2rays(cam, dev)
                rets["scout_loss_data"] = {"points_base": base, "points_target": points.detach(),
                                           "render_mask": mask}
            else:
                p0, rays_d, _ = depths_to_points(cam, median.detach())
                points = p0.detach() + offset
        feats = ingp(points, with_xyz=False)
        ngp = ingp.rgb_decode(feats, torch_F.normalize(rays_d, dim=-1).float())
        ngp = ngp.view(H, W, 3).permute(2, 0, 1) * mask
        rets["ngp_rgb"] = ngp.clone()
        image = image + ngp if mode == "diffuse_ngp" else ngp
    if float(bg_color.sum()) > 0:
        image = image + (1.0 - render_alpha) * bg_color.to(dev).unsqueeze(-1).unsqueeze(-1)
    rets["render"] = image
    if record_transmittance:
        rets.update({"transmittance_avg": trans_avg, "cover_pixels": cover})
    if with_surface:
        rets.update(surface_maps(cam, allmap, getattr(pipe, "depth_ratio", 0.0)))
    return rets


def _render_hybrid(cam, pc, pipe, bg_color, scaling_modifier, ingp, beta, max_intersections, with_surface, mode,
                   decompose_mode, record_transmittance):
    """gaussian_renderer/__init__.py:600-680 (raw SH colours, or the 48
    coefficients, as colors_precomp; the packed level), :958-1000 (the mask,
    and for hybrid_SH_post the per-pixel SH evaluation along the view ray),
    :1013-1046.  The grid is ingp's one level of 3 channels."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings

    if pc.get_features is None or ingp is None:
        raise ValueError(f"mode {mode!r} needs the splats' SH features and the one-level ingp grid")
    if decompose_mode not in DECOMPOSE:
        raise ValueError(f"decompose_mode must be one of {tuple(DECOMPOSE)} (got {decompose_mode!r})")
    rmode = HYBRID_MODES[mode]
    dev = pc.get_xyz.device
    H, W = int(cam.image_height), int(cam.image_width)
    deg = int(pc.active_sh_degree)
    feats = pc.get_features
    K = feats.shape[1]
    shs_view = feats.transpose(1, 2).reshape(-1, 3, K)
    if rmode == 9:
        if K != 16:
            raise ValueError("hybrid_SH_post passes 48 coefficients per splat (SH degree 3 features)")
        colors = shs_view.reshape(-1, 48)
    else:
        campos = _matrix(cam.camera_center, dev).reshape(1, 3)
        d = pc.get_xyz - campos
        colors = eval_sh(deg, shs_view, d / d.norm(dim=1, keepdim=True))
    C = 48 if rmode == 9 else 3
    enc = ingp.hash_encoding
    features, offsets, _, per_level_scale, base_resolution, align_corners, interpolation = enc.get_params()
    host = getattr(enc, "_offsets_host", None)
    if host is not None:
        offsets._nest_host_copy = (offsets._version, np.asarray(host, dtype=np.float64).astype(np.int64))
    gridrange = ingp.gridrange
    gridrange._nest_host_copy = (gridrange._version, ingp._gridrange_host)
    level = (DECOMPOSE[decompose_mode] << 24) | (deg << 16) | (1 << 8)
    raster_settings = GaussianRasterizationSettings(
        image_height=H, image_width=W, tanfovx=math.tan(cam.FoVx * 0.5), tanfovy=math.tan(cam.FoVy * 0.5),
        bg=bg_color, scale_modifier=scaling_modifier, viewmatrix=cam.world_view_transform,
        projmatrix=cam.full_proj_transform, sh_degree=deg, campos=cam.camera_center, prefiltered=False, debug=False,
        beta=beta, if_contract=ingp.contract, record_transmittance=record_transmittance,
        max_intersections=max_intersections)
    hashgrid_settings = HashGridSettings(L=level, S=math.log2(per_level_scale), H=base_resolution,
                                         align_corners=align_corners, interpolation=interpolation,
                                         shape_dims=torch.tensor([0, C, C], dtype=torch.int32))
    rasterizer = GaussianRasterizer(raster_settings=raster_settings, hashgrid_settings=hashgrid_settings)
    means2D = torch.zeros_like(pc.get_xyz)
    image, radii, allmap, trans_avg, cover = rasterizer(
        means3D=pc.get_xyz, means2D=means2D, shs=None, colors_precomp=colors, opacities=pc.get_opacity,
        scales=pc.get_scaling, rotations=pc.get_rotation, homotrans=pc.get_homotrans(),
        ap_level=pc.get_appearance_level, features=features, offsets=offsets, gridrange=gridrange,
        render_mode=rmode)
    render_alpha = allmap[1:2]
    mask = render_alpha > 0
    if rmode == 9:
        rays_d, _ = cam2rays(cam, dev)
        coeffs = image.view(48, -1).permute(1, 0).reshape(-1, 3, 16)
        rgb = torch.clamp_min(eval_sh(deg, coeffs, torch_F.normalize(rays_d, dim=-1)) + 0.5, 0.0)
        image = rgb.view(H, W, 3).permute(2, 0, 1) * mask
    else:
        image = image * mask
    if float(bg_color.sum()) > 0:
        image = image + (1.0 - render_alpha) * bg_color.to(dev).unsqueeze(-1).unsqueeze(-1)
    rets = {"render": image, "viewspace_points": means2D, "visibility_filter": radii > 0, "radii": radii,
            "allmap": allmap}
    if record_transmittance:
        rets.update({"transmittance_avg": trans_avg, "cover_pixels": cover})
    if with_surface:
        rets.update(surface_maps(cam, allmap, getattr(pipe, "depth_ratio", 0.0)))
    return rets


def surface_maps(cam, allmap: torch.Tensor, depth_ratio: float = 0.0) -> dict:
    """The allmap post-processing of gaussian_renderer/__init__.py:763-791:
    world-space normal map, median and expected depth, distortion, the
    pseudo-surface depth (depth_ratio blends expected and median depth) and
    its normal from the back-projected depth map, scaled by alpha."""
    dev = allmap.device
    render_alpha = allmap[1:2]
    wv = _matrix(cam.world_view_transform, dev)
    render_normal = (allmap[2:5].permute(1, 2, 0) @ (wv[:3, :3].T)).permute(2, 0, 1)
    render_depth_median = torch.nan_to_num(allmap[5:6], 0, 0)
    render_depth_expected = torch.nan_to_num(allmap[0:1] / render_alpha, 0, 0)
    render_dist = allmap[6:7]
    surf_depth = render_depth_expected * (1 - depth_ratio) + depth_ratio * render_depth_median
    surf_normal = depth_to_normal(cam, surf_depth).permute(2, 0, 1) * render_alpha.detach()
    return {"rend_alpha": render_alpha, "rend_normal": render_normal, "rend_dist": render_dist,
            "surf_depth": surf_depth, "surf_normal": surf_normal, "gaussian_num": allmap[7:8],
            "depth_expected": render_depth_expected, "depth_median": render_depth_median}


def scene_to_device(scene, device="cuda:0"):
    """(SplatModel, HashINGP) for a synthetic Scene."""
    from gridencoder import GridEncoder

    sp = scene.spec
    dev = torch.device(device)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    pc = SplatModel(t(scene.means), t(scene.scales), t(scene.rotations), t(scene.opacity), t(scene.ap_level),
                    homotrans=t(scene.homotrans))
    enc = GridEncoder(3, sp.L, sp.F, sp.per_level_scale, sp.base_res, sp.log2T).to(dev)
    with torch.no_grad():
        tab = t(scene.table)
        enc.embeddings = torch.nn.Parameter(tab, requires_grad=False)
    mlp = NestMLP(sp.C, sp.mlp_width, sp.mlp_dtype, scene.W1, scene.W2, scene.W3).to(dev)
    ingp = HashINGP(enc, mlp, sp.gridrange, sp.contract)
    return pc, ingp


def render_scene(scene, cam_index=0, device="cuda:0", with_surface=False, max_intersections=0):
    pc, ingp = scene_to_device(scene, device)
    cam = scene.cameras[cam_index]
    bg = torch.tensor(scene.spec.bg, dtype=torch.float32, device=device)
    return render(cam, pc, Pipe(), bg, ingp=ingp, with_surface=with_surface, max_intersections=max_intersections)
