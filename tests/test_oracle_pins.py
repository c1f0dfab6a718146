"""Known-answer pins of the oracle's hash-grid level constants, of multi-level
lookups at grid vertices, of the median-depth rule, and of the surface maps
render() derives from the allmap.

Every expected value here is fixed by the mathematics, not by re-evaluating
the oracle's formula:
  - level resolutions res_l = ceil(H * g^l - 1) + 1 from the exact values of
    H * g^l (integers where g^l is rational; irrational values are at least
    0.0037 from an integer, far outside float32 rounding);
  - dense/hashed splits from (res + 1)^3 <= T;
  - vertex indices g0 + r g1 + r^2 g2 and the xor hash written out as integers;
  - the transmittance sequence 1, 1 - a, (1 - a)^2, ... of stacked splats;
  - planes: expected depth, normals and the normal of the back-projected
    depth map are closed forms.
"""
import math

import numpy as np
import pytest

# res_l for base 16 and growth 2^(7/15) (min_logres 4, max_logres 11,
# hash_encoder/modules.py:172-175): 16 * 2^(7l/15) rounded up; l = 0 and
# l = 15 are exactly 16 and 2048 (scale 15 and 2047)
RES_G16 = [16, 23, 31, 43, 59, 81, 112, 154, 213, 295, 407, 562, 777, 1073, 1483, 2048]
# base 16, growth 1.5: 16 * 1.5^l = 3^l 2^(4-l), integers for l <= 4
RES_G15 = [16, 24, 36, 54, 81, 122, 183, 274]
GROWTH_16 = math.exp((math.log(2 ** 11) - math.log(2 ** 4)) / 15)


def test_level_resolutions_known_answers(oracle):
    """or_level_scale (CR/hashgrid.h:122-124) and the library's level table
    give the exact resolutions of the two growth factors the workloads use."""
    from nest_splat import _lib as NL
    for growth, expect in ((GROWTH_16, RES_G16), (1.5, RES_G15)):
        S = math.log2(growth)
        L = len(expect)
        offs = np.arange(L + 1, dtype=np.int64) * (1 << 19)
        lib_scale, lib_res, _ = NL.hashgrid_levels(L, 2, S, 16, offs)
        for l in range(L):
            sc, res = oracle.level_scale(S, 16, l)
            exact = 16.0 * growth ** l - 1.0
            assert res == expect[l], (growth, l, res)
            assert abs(sc - exact) <= 1e-6 * exact, (growth, l, sc, exact)
            assert lib_res[l] == expect[l] and lib_scale[l] == np.float32(sc), (growth, l)
    assert oracle.level_scale(math.log2(GROWTH_16), 16, 0)[0] == 15.0
    assert oracle.level_scale(math.log2(GROWTH_16), 16, 15)[0] == 2047.0
    # integer scales of the 1.5 growth are exact, not one above
    assert [oracle.level_scale(math.log2(1.5), 16, l)[0] for l in range(5)] == [15.0, 23.0, 35.0, 53.0, 80.0]


@pytest.mark.parametrize("log2T,L,growth,dense", [(14, 8, 1.5, 2), (19, 16, GROWTH_16, 5), (21, 16, GROWTH_16, 7),
                                                  (22, 16, GROWTH_16, 8)])
def test_dense_hashed_split(log2T, L, growth, dense):
    """Levels are dense while (res + 1)^3 <= T (the stride loop of
    get_grid_index, CR/hashgrid.h:7-40); the benchmark grids have dense
    prefixes of 2, 5, 7 and 8 levels."""
    from nest_splat import _lib as NL
    offs = np.arange(L + 1, dtype=np.int64) << log2T
    _, res, hashed = NL.hashgrid_levels(L, 4, math.log2(growth), 16, offs)
    assert hashed == [False] * dense + [True] * (L - dense)
    assert all((r + 1) ** 3 <= (1 << log2T) for r in res[:dense])
    assert (res[dense] + 1) ** 3 > (1 << log2T)


# A 4-level grid with S = 1, H = 2: scale_l = 2^(l+1) - 1 (1, 3, 7, 15),
# res_l = 2, 4, 8, 16.  Level sizes make level 2 hashed, the others dense.
MULTI_S, MULTI_H = 1.0, 2
MULTI_T = {False: [32, 128, 512, 8192], True: [32, 128, 256, 8192]}
# (level, vertex g, expected table row = offsets[level] + index), written out:
#   dense, not aligned: stride r+1 = 3, 5, 9, 17; aligned: stride r = 2, 4, 8, 16
#   hashed: g0 ^ g1*2654435761 ^ g2*805459861 (mod 2^32) mod T
# Without align_corners the cell position is u * scale + 0.5, so the vertices
# reachable from u in [0, 1] have every coordinate in [1, scale].
MULTI_KAT = {
    False: [  # offsets 0, 32, 160, 672, 8864
        (0, (1, 1, 1), 0 + 1 + 1 * 3 + 1 * 9),                   # 13
        (1, (3, 1, 2), 32 + 3 + 1 * 5 + 2 * 25),                 # 90
        (2, (5, 2, 7), 160 + 1820235380 % 512),                  # 276
        (2, (6, 6, 6), 160 + 2504185694 % 512),                  # 510
        (2, (1, 3, 1), 160 + 3936631431 % 512),                  # 295
        (3, (15, 1, 9), 672 + 15 + 1 * 17 + 9 * 289),            # 3305
        (3, (2, 14, 7), 672 + 2 + 14 * 17 + 7 * 289),            # 2935
    ],
    True: [  # offsets 0, 32, 160, 416, 8608
        (1, (3, 1, 2), 32 + 3 + 1 * 4 + 2 * 16),                 # 71
        (2, (5, 2, 7), 160 + 1820235380 % 256),                  # 276
        (2, (0, 3, 1), 160 + 3936631430 % 256),                  # 294
        (3, (15, 0, 9), 416 + 15 + 0 * 16 + 9 * 256),            # 2735
        (3, (7, 7, 7), 416 + 7 + 7 * 16 + 7 * 256),              # 2327
    ],
}


def _vertex_coord(scale: np.float32, g: int, align: bool):
    """A float32 u in [0, 1] whose cell position u * scale (+ 0.5) is exactly
    the integer g, so corner 0 has weight 1 and the other seven weight 0."""
    off = np.float32(0.0 if align else 0.5)
    u0 = np.float32((g - float(off)) / float(scale))
    cands = [u0]
    up = dn = u0
    for _ in range(256):
        up = np.nextafter(up, np.float32(2))
        dn = np.nextafter(dn, np.float32(-1))
        cands += [up, dn]
    for u in cands:
        if 0 <= u <= 1 and np.float32(np.float32(u * scale) + off) == np.float32(g):
            return u
    return None


@pytest.mark.parametrize("align", [False, True])
def test_multilevel_vertex_known_answers(oracle, align):
    """A table holding its own row numbers (channel 0) and their negatives
    (channel 1), queried exactly at a vertex of level l, returns
    offsets[l] + index at level l: the per-level scale, the stride loop with
    r+1 (r when align_corners), the hash and the level's base row.  Both the
    render's query_feature and the GridEncoder forward are checked."""
    T = MULTI_T[align]
    offs = np.concatenate([[0], np.cumsum(T)]).astype(np.int32)
    rows = np.arange(offs[-1], dtype=np.float32)
    table = np.stack([rows, -rows], 1)
    L, F = 4, 2
    grid = oracle.make_grid(L, F, MULTI_S, MULTI_H, offs, table, (0.0, 1.0), False, align)
    for level, g, row in MULTI_KAT[align]:
        scale, _ = oracle.level_scale(MULTI_S, MULTI_H, level)
        assert scale == 2.0 ** (level + 1) - 1
        u = [_vertex_coord(np.float32(scale), gd, align) for gd in g]
        assert all(v is not None for v in u), (level, g)
        u = np.array(u, np.float32)
        feat = oracle.query_feature(grid, u, 24, L * F)
        assert feat[level * F] == row and feat[level * F + 1] == -row, (level, g, feat[level * F], row)
        enc = oracle.grid_encode(grid, u[None, :])[0]
        assert enc[level * F] == row and enc[level * F + 1] == -row
        # the appearance cap drops exactly the levels at or past it
        capped = oracle.query_feature(grid, u, level, L * F)
        assert not capped[level * F:].any()


# ------------------------------------------------------------------ median

def _stack_scene(opacities, depths, W=63, H=47):
    """Splats facing a camera on the -y axis, centred on the ray of the
    principal pixel ((W-1)/2, (H-1)/2), at view depths `depths`."""
    from nest_splat.camera import look_at
    cam = look_at((0.0, -3.0, 0.0), (0.0, 0.0, 0.0), 50.0, W, H)
    n = len(depths)
    means = np.zeros((n, 3), np.float32)
    means[:, 1] = np.asarray(depths, np.float32) - 3.0
    q = np.tile(np.array([np.cos(np.pi / 4), np.sin(np.pi / 4), 0, 0], np.float32), (n, 1))
    scales = np.full((n, 2), 0.2, np.float32)
    opac = np.asarray(opacities, np.float32).reshape(n, 1)
    return cam, means, scales, q, opac


@pytest.mark.parametrize("alpha,median_hit", [(0.3, 2), (0.2, 4), (0.5, 1), (0.6, 1)])
def test_median_depth_closed_form(oracle, alpha, median_hit):
    """At the centre pixel every splat has G = 1, alpha = opacity, and T runs
    1, 1 - a, (1 - a)^2, ...; the median is the last hit taken while T > 0.5
    (CR/forward.cu:1917-1920), counted in splats visited, rejected ones
    included: with a rejected splat in front, the median contributor is
    median_hit + 1 and the median depth is that hit's depth."""
    depths = [2.0] + [2.5 + 0.25 * k for k in range(8)]
    opac = [0.001] + [alpha] * 8                      # 0.001 < 1/255: visited, rejected
    cam, means, scales, q, opac = _stack_scene(opac, depths)
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(means, scales, q, opac, cam.world_view_transform, cam.full_proj_transform, W, H)
    assert np.all(pre["radii"] > 0)
    b = oracle.binning(pre, W, H)
    r = oracle.render(pre, b, W, H, 3, None, colors=np.ones((len(depths), 3), np.float32))
    cx, cy = (W - 1) // 2, (H - 1) // 2
    # closed-form transmittance sequence and the median hit
    a = np.float32(alpha)
    T, hits, med = np.float32(1), 0, None
    for k in range(8):
        if T * (np.float32(1) - a) < np.float32(1e-4):
            break
        if T > 0.5:
            med = k + 1
        T = np.float32(T * (np.float32(1) - a))
        hits += 1
    assert med == median_hit
    assert r["n_contrib"][1, cy, cx] == median_hit + 1
    assert r["others"][5, cy, cx] == pytest.approx(depths[median_hit], abs=1e-5)
    assert r["others"][7, cy, cx] == hits
    assert r["others"][1, cy, cx] == np.float32(1) - T


def test_median_depth_of_pixels_without_hits(oracle):
    """A pixel with no hit keeps median depth 0 and median contributor -1,
    stored through the saturating float->uint32 conversion as 0."""
    cam, means, scales, q, opac = _stack_scene([0.5], [3.0])
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(means, scales, q, opac, cam.world_view_transform, cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    r = oracle.render(pre, b, W, H, 3, None, colors=np.ones((1, 3), np.float32))
    empty = r["others"][7] == 0
    assert empty.any()
    assert not r["others"][5][empty].any() and not r["n_contrib"][1][empty].any()


# ----------------------------------------------------------- surface maps

def _plane_scene(normal_world, dist=10.0, W=96, H=72, opacity=0.99, sigma=4.0):
    """One large splat whose plane has the given world normal and passes
    through the point at `dist` on the camera's axis (camera at the origin
    looking along +y).  Its 4-sigma disk stays in front of the camera (the
    projected bounding box of 2D surfels needs that)."""
    from nest_splat.camera import look_at
    cam = look_at((0.0, 0.0, 0.0), (0.0, 1.0, 0.0), 50.0, W, H)
    n = np.asarray(normal_world, np.float64)
    n = n / np.linalg.norm(n)
    # rotation whose third column is n
    a = np.array([1.0, 0.0, 0.0]) if abs(n[0]) < 0.9 else np.array([0.0, 0.0, 1.0])
    t0 = np.cross(n, a)
    t0 /= np.linalg.norm(t0)
    t1 = np.cross(n, t0)
    R = np.stack([t0, t1, n], 1)
    w = math.sqrt(max(0.0, 1 + R[0, 0] + R[1, 1] + R[2, 2])) / 2
    q = np.array([w, (R[2, 1] - R[1, 2]) / (4 * w), (R[0, 2] - R[2, 0]) / (4 * w), (R[1, 0] - R[0, 1]) / (4 * w)])
    means = np.array([[0.0, dist, 0.0]], np.float32)
    return cam, means, np.full((1, 2), sigma, np.float32), q[None, :].astype(np.float32), \
        np.full((1, 1), opacity, np.float32), n


@pytest.mark.parametrize("normal", [(0.0, -1.0, 0.0), (0.3, -1.0, 0.2)])
def test_surface_maps_closed_form(oracle, normal):
    """render()'s surface outputs (gaussian_renderer/__init__.py:763-791,
    utils/point_utils.py:10-60) on a single plane, from the oracle's allmap:
      rend_normal = alpha * n (world normal facing the camera);
      surf_depth (expected depth) = the view depth of the ray/plane hit,
        along rays through pixel (x, y) with principal point ((W-1)/2, (H-1)/2);
      surf_normal = alpha * n', the normal of the plane the back-projection
        with principal point (W/2, H/2) maps it to: X' = X - Z/(2 fx),
        Y' = Y - Z/(2 fy), so n' = n + (0, 0, (n_x/fx + n_y/fy)/2) in view
        space, normalised."""
    import torch

    from nest_splat.renderer import surface_maps
    cam, means, scales, q, opac, n = _plane_scene(normal)
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(means, scales, q, opac, cam.world_view_transform, cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    r = oracle.render(pre, b, W, H, 3, None, colors=np.ones((1, 3), np.float32))
    allmap = torch.from_numpy(r["others"])
    out = surface_maps(cam, allmap, depth_ratio=0.0)
    alpha = r["others"][1]
    cov = alpha > 0.05
    assert cov.mean() > 0.9
    V = cam.world_view_transform.astype(np.float64)          # p_view = [p, 1] @ V
    R = V[:3, :3]
    if n @ (np.array([0.0, 0.0, 0.0]) - means[0]) < 0:       # face the camera (at the origin)
        n = -n
    rn = out["rend_normal"].numpy()
    np.testing.assert_allclose(rn[:, cov] / alpha[cov], np.broadcast_to(n[:, None], (3, cov.sum())), atol=2e-5)
    # expected depth: view depth of the ray/plane intersection, rasterizer's pixel model
    fx = W / (2 * cam.tanfovx)
    fy = H / (2 * cam.tanfovy)
    nv = n @ R                                               # view-space normal
    pv = np.concatenate([means[0].astype(np.float64), [1.0]]) @ V
    ys, xs = np.mgrid[0:H, 0:W]
    dirs = np.stack([(xs - (W - 1) / 2) / fx, (ys - (H - 1) / 2) / fy, np.ones_like(xs, float)], -1)
    z = (nv @ pv[:3]) / (dirs @ nv)
    sd = out["surf_depth"].numpy()[0]
    np.testing.assert_allclose(sd[cov], z[cov], rtol=2e-5)
    # surface normal of the back-projected depth map (interior pixels whose
    # 4-neighbourhood is covered)
    npv = nv + np.array([0.0, 0.0, (nv[0] / fx + nv[1] / fy) / 2])
    npv /= np.linalg.norm(npv)
    if npv @ (-pv[:3]) < 0:
        npv = -npv
    nw = R @ npv                                             # back to world (R orthonormal)
    inner = np.zeros_like(cov)
    inner[1:-1, 1:-1] = cov[1:-1, 1:-1] & cov[2:, 1:-1] & cov[:-2, 1:-1] & cov[1:-1, 2:] & cov[1:-1, :-2]
    sn = out["surf_normal"].numpy()
    # 4e-5 separates n' from n (they differ by 1.3e-4 on the tilted plane)
    np.testing.assert_allclose(sn[:, inner] / alpha[inner], np.broadcast_to(nw[:, None], (3, inner.sum())),
                               atol=4e-5)
    assert not sn[:, 0, :].any() and not sn[:, :, 0].any()   # one-pixel border stays zero
    # the principal-point mismatch is visible for the tilted plane only
    if abs(nv[0]) + abs(nv[1]) > 1e-3:
        assert np.abs(npv - nv / np.linalg.norm(nv)).max() > 1e-4
