"""Seeded synthetic scenes for the five benchmark workloads.

RNG: numpy Generator(PCG64(seed)); draw order centers -> log-scales ->
quaternions -> opacity logits -> (RVQ codebooks, indices) -> hash table -> MLP
weights.  Activations follow scene/gaussian_model.py:26-41 (exp, normalize,
sigmoid) and homotrans follows utils/general_utils.py:78-113 (build_rotation,
build_H), all in float32 numpy so that the GPU path and the oracle receive the
same bits.  ap_level is 24.0 for every splat (scene/gaussian_model.py:373-376).
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from .camera import Camera, look_at, orbit_cameras


@dataclass
class SceneSpec:
    name: str
    seed: int
    P: int
    W: int
    H: int
    layout: str                      # "cube" | "shell" | "ball_unbounded" | "shells"
    log_scale_mu: float
    log_scale_sigma: float
    opacity_mu: float
    opacity_sigma: float
    L: int
    F: int
    log2T: int
    base_res: int
    per_level_scale: float
    gridrange: tuple
    contract: bool
    table_dtype: str                 # "f32" | "f16"
    mlp_width: int
    mlp_dtype: str                   # "f32" | "f16" | "bf16"
    bg: tuple = (0.0, 0.0, 0.0)
    fovx_deg: float = 50.0
    cam_dist: float = 3.0
    n_cams: int = 1
    rvq: bool = False
    rvq_stages: int = 4
    rvq_codebook: int = 4096
    table_init: float = 0.1

    @property
    def C(self) -> int:
        return self.L * self.F

    @property
    def S(self) -> float:
        return math.log2(self.per_level_scale)

    def scaled(self, **kw) -> "SceneSpec":
        return dataclasses.replace(self, **kw)


GROWTH_16 = math.exp((math.log(2 ** 11) - math.log(2 ** 4)) / 15)  # min_logres 4, max_logres 11

SPECS = {
    # CPU-runnable plumbing scene: 2000 splats in a cube, 128x128
    "cfg1": SceneSpec("cfg1", 20261, 2000, 128, 128, "cube", -3.0, 0.3, 0.0, 1.0,
                      8, 2, 14, 16, 1.5, (-1.5, 1.5), False, "f32", 64, "f32"),
    # object-scale sphere shell: 100k splats, 800x800
    "cfg2": SceneSpec("cfg2", 20262, 100_000, 800, 800, "shell", -4.5, 0.3, 1.0, 1.0,
                      16, 2, 19, 16, GROWTH_16, (-1.5, 1.5), False, "f32", 64, "f16",
                      bg=(1.0, 1.0, 1.0)),
    # unbounded 1M-splat scene, the headline workload; scales and opacities
    # as in cfg2, camera at distance 2.6: the oracle measures a mean of 41.6
    # accepted hits per pixel (every pixel is covered)
    "cfg3": SceneSpec("cfg3", 20263, 1_000_000, 1600, 1064, "ball_unbounded", -4.5, 0.3, 1.0, 1.0,
                      16, 4, 21, 16, GROWTH_16, (-1.0, 1.0), True, "f32", 64, "bf16",
                      cam_dist=2.6),
    # RVQ-compressed attributes: 500k splats, 800x800
    "cfg4": SceneSpec("cfg4", 20264, 500_000, 800, 800, "shell", -4.5, 0.3, 1.0, 1.0,
                      16, 2, 19, 16, GROWTH_16, (-1.5, 1.5), False, "f32", 64, "f16",
                      bg=(1.0, 1.0, 1.0), rvq=True),
    # stress scene: 4M splats in 5 shells, 8 orbit cameras at 1920x1080
    "cfg5": SceneSpec("cfg5", 20265, 4_000_000, 1920, 1080, "shells", -4.5, 0.3, -3.0, 1.0,
                      16, 4, 22, 16, GROWTH_16, (-3.0, 3.0), False, "f16", 128, "bf16",
                      cam_dist=4.5, n_cams=8),
}

# RVQ dequantisation bias per attribute: decoded = bias + ordered stage sum.
RVQ_BIAS = {"scale": (-4.5, -4.5), "rotation": (1.0, 0.0, 0.0, 0.0), "opacity": (1.0,)}
RVQ_DIMS = {"scale": 2, "rotation": 4, "opacity": 1}


def _random_unit(rng, n):
    v = rng.standard_normal((n, 3))
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def _quat_from_normal(nrm: np.ndarray, rng) -> np.ndarray:
    """Quaternions (w,x,y,z) whose rotation maps +z onto nrm, with a random
    spin about the normal, so the surfel's third axis is the surface normal."""
    n = nrm.shape[0]
    z = np.array([0.0, 0.0, 1.0])
    axis = np.cross(np.broadcast_to(z, nrm.shape), nrm)
    s = np.linalg.norm(axis, axis=1)
    c = nrm[:, 2]
    ang = np.arctan2(s, c)
    axis = np.where(s[:, None] > 1e-12, axis / np.maximum(s, 1e-12)[:, None], np.array([1.0, 0.0, 0.0]))
    q1 = np.concatenate([np.cos(ang / 2)[:, None], axis * np.sin(ang / 2)[:, None]], axis=1)
    spin = rng.uniform(0, 2 * np.pi, n)
    q2 = np.stack([np.cos(spin / 2), np.zeros(n), np.zeros(n), np.sin(spin / 2)], axis=1)
    # q = q1 * q2 (apply spin about z first)
    w1, x1, y1, z1 = q1.T
    w2, x2, y2, z2 = q2.T
    return np.stack([w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2,
                     w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                     w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2,
                     w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2], axis=1)


def build_rotation_np(q: np.ndarray) -> np.ndarray:
    """utils/general_utils.py:78-99 in float32."""
    q = q.astype(np.float32)
    norm = np.sqrt(q[:, 0] * q[:, 0] + q[:, 1] * q[:, 1] + q[:, 2] * q[:, 2] + q[:, 3] * q[:, 3])
    q = q / norm[:, None]
    r, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    R = np.zeros((q.shape[0], 3, 3), dtype=np.float32)
    one, two = np.float32(1), np.float32(2)
    R[:, 0, 0] = one - two * (y * y + z * z)
    R[:, 0, 1] = two * (x * y - r * z)
    R[:, 0, 2] = two * (x * z + r * y)
    R[:, 1, 0] = two * (x * y + r * z)
    R[:, 1, 1] = one - two * (x * x + z * z)
    R[:, 1, 2] = two * (y * z - r * x)
    R[:, 2, 0] = two * (x * z - r * y)
    R[:, 2, 1] = two * (y * z + r * x)
    R[:, 2, 2] = one - two * (x * x + y * y)
    return R


def build_homotrans_np(q: np.ndarray, scales: np.ndarray, xyz: np.ndarray) -> np.ndarray:
    """utils/general_utils.py:101-113: [[R diag(sx, sy, 0), xyz], [0, 0, 0, 1]]."""
    R = build_rotation_np(q)
    P = q.shape[0]
    s = np.zeros((P, 1, 3), dtype=np.float32)
    s[:, 0, :2] = scales
    h = np.zeros((P, 4, 4), dtype=np.float32)
    h[:, :3, :3] = s * R
    h[:, :3, 3] = xyz
    h[:, 3, 3] = 1.0
    return h


def rvq_decode_np(cb: np.ndarray, idx: np.ndarray, bias) -> np.ndarray:
    """bias + (((cb0[i0] + cb1[i1]) + cb2[i2]) + cb3[i3]) in float32."""
    S = cb.shape[0]
    v = cb[0][idx[:, 0].astype(np.int64)]
    for s in range(1, S):
        v = v + cb[s][idx[:, s].astype(np.int64)]
    return (np.asarray(bias, dtype=np.float32)[None, :] + v).astype(np.float32)


def hash_offsets(L: int, log2T: int) -> np.ndarray:
    """Uniform level offsets l * 2^log2T (gridencoder/grid.py:120-130)."""
    return (np.arange(L + 1, dtype=np.int64) * (1 << log2T)).astype(np.int32)


@dataclass
class Scene:
    spec: SceneSpec
    means: np.ndarray
    scales: np.ndarray
    rotations: np.ndarray
    opacity: np.ndarray          # [P, 1]
    homotrans: np.ndarray        # [P, 4, 4]
    ap_level: np.ndarray         # [P, 1]
    table: np.ndarray            # [L*T, F] float32 or float16
    offsets: np.ndarray          # int32 [L+1]
    W1: np.ndarray
    W2: np.ndarray
    W3: np.ndarray
    cameras: List[Camera]
    rvq_codebooks: Optional[dict] = None   # attr -> float32 [S, K, dim]
    rvq_indices: Optional[dict] = None     # attr -> uint16 [P, S]


def _centers(spec: SceneSpec, rng) -> np.ndarray:
    P = spec.P
    if spec.layout == "cube":
        return rng.uniform(-1.0, 1.0, (P, 3))
    if spec.layout == "shell":
        d = _random_unit(rng, P)
        r = 1.0 + 0.02 * rng.standard_normal(P)
        return d * r[:, None]
    if spec.layout == "ball_unbounded":
        n_in = int(round(0.7 * P))
        d = _random_unit(rng, P)
        u = rng.uniform(0.0, 1.0, P)
        r = np.empty(P)
        r[:n_in] = np.cbrt(u[:n_in])
        r[n_in:] = 1.0 + 19.0 * u[n_in:]
        return d * r[:, None]
    if spec.layout == "shells":
        d = _random_unit(rng, P)
        shell = rng.integers(0, 5, P)
        r = 0.5 + 0.5 * shell + 0.02 * rng.standard_normal(P)
        return d * r[:, None]
    raise ValueError(spec.layout)


def make_scene(spec: SceneSpec, with_table: bool = True) -> Scene:
    rng = np.random.Generator(np.random.PCG64(spec.seed))
    P = spec.P
    means = _centers(spec, rng)
    log_scales = spec.log_scale_mu + spec.log_scale_sigma * rng.standard_normal((P, 2))
    if spec.layout in ("shell", "shells"):
        nrm = means / np.linalg.norm(means, axis=1, keepdims=True)
        quats = _quat_from_normal(nrm, rng)
    else:
        quats = rng.standard_normal((P, 4))
        quats /= np.linalg.norm(quats, axis=1, keepdims=True)
    op_logit = spec.opacity_mu + spec.opacity_sigma * rng.standard_normal(P)

    cbs = idxs = None
    if spec.rvq:
        cbs, idxs = {}, {}
        for a in ("scale", "rotation", "opacity"):
            cbs[a] = (0.1 * rng.standard_normal((spec.rvq_stages, spec.rvq_codebook, RVQ_DIMS[a]))).astype(np.float32)
        for a in ("scale", "rotation", "opacity"):
            idxs[a] = rng.integers(0, spec.rvq_codebook, (P, spec.rvq_stages)).astype(np.uint16)

    means32 = means.astype(np.float32)
    if spec.rvq:
        dec = {a: rvq_decode_np(cbs[a], idxs[a], RVQ_BIAS[a]) for a in cbs}
        log_scales, quats, op_logit = dec["scale"], dec["rotation"], dec["opacity"][:, 0]
    scales32 = np.exp(log_scales.astype(np.float32))
    rot32 = quats.astype(np.float32)
    rot32 = rot32 / np.maximum(np.linalg.norm(rot32, axis=1, keepdims=True), np.float32(1e-12))
    opac32 = (np.float32(1) / (np.float32(1) + np.exp(-op_logit.astype(np.float32))))[:, None]

    T = 1 << spec.log2T
    if with_table:
        tab = rng.uniform(-spec.table_init, spec.table_init, (spec.L * T, spec.F)).astype(np.float32)
        if spec.table_dtype == "f16":
            tab = tab.astype(np.float16)
    else:
        tab = np.zeros((0, spec.F), dtype=np.float32)
        rng.uniform(size=1)

    def xavier(o, i):
        a = math.sqrt(6.0 / (i + o))
        return rng.uniform(-a, a, (o, i)).astype(np.float32)

    N = spec.mlp_width
    W1 = xavier(N, spec.C + 16)
    W2 = xavier(N, N)
    W3 = xavier(3, N)

    if spec.n_cams == 1:
        cams = [look_at((0.0, -spec.cam_dist, 0.35 * spec.cam_dist), (0, 0, 0), spec.fovx_deg, spec.W, spec.H)]
    else:
        cams = orbit_cameras(spec.n_cams, spec.cam_dist, 0.3 * spec.cam_dist, spec.fovx_deg, spec.W, spec.H)

    homo = build_homotrans_np(rot32, scales32, means32)
    return Scene(spec, means32, scales32, rot32, opac32, homo,
                 np.full((P, 1), 24.0, dtype=np.float32), tab, hash_offsets(spec.L, spec.log2T),
                 W1, W2, W3, cams, cbs, idxs)


def get_spec(config: str, **overrides) -> SceneSpec:
    s = SPECS[config]
    return s.scaled(**overrides) if overrides else s
