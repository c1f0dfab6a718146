"""Pinhole cameras in the reference's matrix conventions.

Follows utils/graphics_utils.py:38-71 (getWorld2View2, getProjectionMatrix) and
scene/cameras.py:55-66 (world_view_transform, full_proj_transform,
camera_center): row-vector convention, matrices stored transposed, znear 0.01,
zfar 100.  ``view_ray_matrix`` restates utils/point_utils.py:31-46 (cam2rays),
whose principal point is (W/2, H/2), unlike the rasterizer's (W-1)/2.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def get_world2view2(R: np.ndarray, t: np.ndarray) -> np.ndarray:
    """utils/graphics_utils.py:38-49 with translate 0 and scale 1."""
    Rt = np.zeros((4, 4))
    Rt[:3, :3] = R.transpose()
    Rt[:3, 3] = t
    Rt[3, 3] = 1.0
    return Rt


def get_projection_matrix(znear: float, zfar: float, fovX: float, fovY: float) -> np.ndarray:
    """utils/graphics_utils.py:51-71."""
    tanHalfFovY = math.tan(fovY / 2)
    tanHalfFovX = math.tan(fovX / 2)
    top = tanHalfFovY * znear
    bottom = -top
    right = tanHalfFovX * znear
    left = -right
    P = np.zeros((4, 4))
    P[0, 0] = 2.0 * znear / (right - left)
    P[1, 1] = 2.0 * znear / (top - bottom)
    P[0, 2] = (right + left) / (right - left)
    P[1, 2] = (top + bottom) / (top - bottom)
    P[3, 2] = 1.0
    P[2, 2] = zfar / (zfar - znear)
    P[2, 3] = -(zfar * znear) / (zfar - znear)
    return P


@dataclass
class Camera:
    """The camera fields the forward render reads (scene/cameras.py:17-66)."""

    image_width: int
    image_height: int
    FoVx: float
    FoVy: float
    world_view_transform: np.ndarray  # float32 [4,4], transposed world->view
    projection_matrix: np.ndarray     # float32 [4,4], transposed
    full_proj_transform: np.ndarray   # float32 [4,4]
    camera_center: np.ndarray         # float32 [3]
    znear: float = 0.01
    zfar: float = 100.0

    @property
    def tanfovx(self) -> float:
        return math.tan(self.FoVx * 0.5)

    @property
    def tanfovy(self) -> float:
        return math.tan(self.FoVy * 0.5)


def camera_from_rt(R: np.ndarray, t: np.ndarray, fovx: float, W: int, H: int) -> Camera:
    focal = W / (2.0 * math.tan(fovx / 2.0))
    fovy = 2.0 * math.atan(H / (2.0 * focal))
    wv = get_world2view2(R, t).T
    pm = get_projection_matrix(0.01, 100.0, fovx, fovy).T
    wv32 = wv.astype(np.float32)
    pm32 = pm.astype(np.float32)
    full = (wv32.astype(np.float64) @ pm32.astype(np.float64)).astype(np.float32)
    center = np.linalg.inv(wv32.astype(np.float64))[3, :3].astype(np.float32)
    return Camera(W, H, fovx, fovy, wv32, pm32, full, center)


def look_at(eye, target, fovx_deg: float, W: int, H: int, up=(0.0, 0.0, 1.0)) -> Camera:
    """A camera at ``eye`` looking at ``target``: x right, y down, z forward."""
    eye = np.asarray(eye, dtype=np.float64)
    target = np.asarray(target, dtype=np.float64)
    up = np.asarray(up, dtype=np.float64)
    z = target - eye
    z /= np.linalg.norm(z)
    x = np.cross(-up, z)
    if np.linalg.norm(x) < 1e-8:
        x = np.cross(np.array([0.0, 1.0, 0.0]), z)
    x /= np.linalg.norm(x)
    y = np.cross(z, x)
    R = np.stack([x, y, z], axis=1)  # camera-to-world rotation, columns = axes
    t = -R.T @ eye
    return camera_from_rt(R, t, math.radians(fovx_deg), W, H)


def orbit_cameras(n: int, radius: float, height: float, fovx_deg: float, W: int, H: int):
    cams = []
    for k in range(n):
        a = 2.0 * math.pi * k / n
        eye = (radius * math.cos(a), radius * math.sin(a), height)
        cams.append(look_at(eye, (0.0, 0.0, 0.0), fovx_deg, W, H))
    return cams


def view_ray_matrix(cam: Camera) -> np.ndarray:
    """3x3 M with rays_d(x, y) = (x, y, 1) @ M, as cam2rays builds them
    (utils/point_utils.py:31-46): M = inv(K)^T @ R_c2w^T with principal point
    (W/2, H/2).  Evaluated in float64 and rounded once to float32."""
    W, H = cam.image_width, cam.image_height
    wv = cam.world_view_transform.astype(np.float64)
    c2w = np.linalg.inv(wv.T)
    ndc2pix = np.array([[W / 2, 0, 0, W / 2],
                        [0, H / 2, 0, H / 2],
                        [0, 0, 0, 1]], dtype=np.float64).T
    projection_matrix = c2w.T @ cam.full_proj_transform.astype(np.float64)
    intrins = (projection_matrix @ ndc2pix)[:3, :3].T
    M = np.linalg.inv(intrins).T @ c2w[:3, :3].T
    return M.astype(np.float32)
