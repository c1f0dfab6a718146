"""GPU parity of the plain 2DGS colour path with colours evaluated from SH in
preprocess (computeColorFromSH, CR/forward.cu:21-72, :417-424) and of
markVisible (DSR/rasterize_points.cu:452-470), against the oracle: the SH
colours, clamp flags, rendered colour and allmap bit for bit."""
import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("name,deg,M", [("cfg1", 3, 16), ("cfg1", 0, 1), ("shell_small", 1, 16), ("shell_small", 2, 9)])
def test_sh_colour_path_matches_oracle(oracle, name, deg, M):
    from nest_splat import rasterizer as rz
    sc = scene(name)
    sp = sc.spec
    cam = sc.cameras[0]
    rng = np.random.default_rng(deg * 10 + M)
    shs = rng.normal(0, 0.6, (sp.P, M, 3)).astype(np.float32)
    print(f"[case] {name} deg={deg} M={M} P={sp.P}", flush=True)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center)
    grid = rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               channels=3, shs=_t(shs), sh_degree=deg)
    torch.cuda.synchronize()
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    rgb, clamped = oracle.sh_colors(pre, sc.means, np.asarray(cam.camera_center, np.float32), shs, deg)
    ga = rz.geometry_arrays(res, sp.P)
    vis = pre["radii"] > 0
    assert vis.sum() > 0
    np.testing.assert_array_equal(ga["rgb"].cpu().numpy()[vis], rgb[vis])
    np.testing.assert_array_equal(ga["clamped"].cpu().numpy()[vis], clamped[vis])
    assert clamped[vis].any(), "the coefficients should clamp some channels"
    b = oracle.binning(pre, W, H)
    r = oracle.render(pre, b, W, H, 3, None, colors=rgb)
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])
    np.testing.assert_array_equal(res.others.cpu().numpy()[:8], r["others"][:8])


def test_drop_in_sh_colour_call(oracle):
    """GaussianRasterizer.forward(shs=...) with L == 0, as render() calls it
    for the colour warm-up (GR:114-120), equals the direct call."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    from nest_splat import rasterizer as rz
    sc = scene("cfg1")
    sp = sc.spec
    cam = sc.cameras[0]
    shs = np.random.default_rng(5).normal(0, 0.5, (sp.P, 16, 3)).astype(np.float32)
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, _t(cam.world_view_transform),
                                       _t(cam.full_proj_transform), 3, _t(cam.camera_center), False, False, 0.0, False,
                                       False)
    hs = HashGridSettings(0, 0.0, 0, False, 0, torch.tensor([0, 3, 3], dtype=torch.int32))
    color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(means3D=_t(sc.means), means2D=None,
                                                           opacities=_t(sc.opacity), shs=_t(shs),
                                                           scales=_t(sc.scales), rotations=_t(sc.rotations))
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center)
    grid = rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               channels=3, shs=_t(shs), sh_degree=3)
    np.testing.assert_array_equal(color.cpu().numpy(), res.color.cpu().numpy())
    np.testing.assert_array_equal(allmap.cpu().numpy(), res.others.cpu().numpy())
    # non-RGB output with SH colours is refused, as the reference throws
    hs5 = hs._replace(shape_dims=torch.tensor([0, 5, 5], dtype=torch.int32))
    with pytest.raises(RuntimeError):
        GaussianRasterizer(rs, hs5)(means3D=_t(sc.means), means2D=None, opacities=_t(sc.opacity), shs=_t(shs),
                                    scales=_t(sc.scales), rotations=_t(sc.rotations))


def test_mark_visible_matches_oracle(oracle):
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("shell_small")
    cam = sc.cameras[0]
    rng = np.random.default_rng(11)
    pts = np.concatenate([sc.means, rng.uniform(-6, 6, (4000, 3)).astype(np.float32)])
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, _t(cam.world_view_transform),
                                       _t(cam.full_proj_transform), 0, _t(cam.camera_center), False, False, 0.0, False,
                                       False)
    vis = GaussianRasterizer(rs, HashGridSettings(0, 0.0, 0, False, 0, torch.empty(0))).markVisible(_t(pts))
    assert vis.dtype == torch.bool and vis.shape == (pts.shape[0],)
    ref = oracle.mark_visible(pts, cam.world_view_transform)
    np.testing.assert_array_equal(vis.cpu().numpy(), ref)
    assert ref.any() and (~ref).any()
    # agrees with the preprocess near cull: every splat preprocess keeps is visible
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, cam.image_width, cam.image_height)
    assert ref[: sc.spec.P][pre["radii"] > 0].all()
    assert GaussianRasterizer(rs, HashGridSettings(0, 0.0, 0, False, 0, torch.empty(0))).markVisible(
        torch.zeros((0, 3), device=DEV)).numel() == 0


def test_build_homotrans_bit_exact():
    """nest_build_homotrans against the reference's torch expressions
    (build_H(build_rotation(r), s, xyz), utils/general_utils.py:78-113) on the
    GPU and their float32 numpy restatement: unnormalised quaternions of mixed
    sign, ragged P, column 2 keeping the sign of 0 * R."""
    from nest_splat import rasterizer as rz
    from nest_splat.renderer import build_H, build_rotation
    from nest_splat.scene import build_homotrans_np
    rng = np.random.default_rng(19)
    P = 100_003
    q = (rng.standard_normal((P, 4)) * rng.uniform(0.1, 3.0, (P, 1))).astype(np.float32)
    s = np.exp(rng.normal(-4, 1, (P, 2))).astype(np.float32)
    x = rng.uniform(-20, 20, (P, 3)).astype(np.float32)
    got = rz.build_homotrans(_t(q), _t(s), _t(x))
    want = build_H(build_rotation(_t(q)), _t(s), _t(x))
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    np.testing.assert_array_equal(g.view(np.uint32), want.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(g.view(np.uint32), build_homotrans_np(q, s, x).view(np.uint32))
    assert np.signbit(g[:, :3, 2]).any()
    assert rz.build_homotrans(torch.zeros((0, 4), device=DEV), torch.zeros((0, 2), device=DEV),
                              torch.zeros((0, 3), device=DEV)).shape == (0, 4, 4)
