"""The drop-in call surface on the GPU: GaussianRasterizer.forward as the
reference's render() calls it, the render() counterpart's output dict, the
RVQ-compressed scene end to end, and error behaviour."""
import math

import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_render_dict_matches_oracle(oracle):
    from nest_splat import renderer
    sc = scene("shell_small")
    out = renderer.render_scene(sc, with_surface=True)
    torch.cuda.synchronize()
    ref = oracle.render_scene(sc)
    np.testing.assert_array_equal(out["allmap"].cpu().numpy(), ref["others"])
    np.testing.assert_array_equal(out["features"].cpu().numpy(), ref["color"])
    np.testing.assert_allclose(out["render"].cpu().numpy(), ref["rgb"], atol=1e-3, rtol=0)
    np.testing.assert_array_equal(out["radii"].cpu().numpy(), ref["pre"]["radii"])
    for k in ("render", "viewspace_points", "visibility_filter", "radii", "rend_alpha", "rend_normal", "rend_dist",
              "surf_depth", "surf_normal", "gaussian_num", "depth_expected", "depth_median"):
        assert k in out, k
    alpha = ref["others"][1]
    exp = np.nan_to_num(ref["others"][0] / alpha, nan=0.0, posinf=0.0, neginf=0.0)
    np.testing.assert_allclose(out["depth_expected"].cpu().numpy()[0], exp, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(out["gaussian_num"].cpu().numpy()[0], ref["others"][7])


def test_drop_in_rasterizer_call(oracle):
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("cfg1")
    sp = sc.spec
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, t(cam.world_view_transform),
                                       t(cam.full_proj_transform), 3, t(cam.camera_center), False, False, 0.0,
                                       sp.contract, False)
    hs = HashGridSettings(sp.L, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                          torch.tensor([0, sp.C, sp.C], dtype=torch.int32, device=DEV))
    r = GaussianRasterizer(rs, hs)
    color, radii, allmap, trans, cover = r(means3D=t(sc.means), means2D=torch.zeros(sp.P, 3, device=DEV),
                                           opacities=t(sc.opacity), shs=torch.zeros(sp.P, 16, 3, device=DEV),
                                           scales=t(sc.scales), rotations=t(sc.rotations), homotrans=t(sc.homotrans),
                                           ap_level=t(sc.ap_level), features=t(sc.table), offsets=t(sc.offsets),
                                           gridrange=t(np.asarray(sp.gridrange, np.float32)))
    ref = oracle.render_scene(sc, with_mlp=False)
    assert color.shape == (sp.C, sp.H, sp.W) and allmap.shape == (14, sp.H, sp.W) and radii.dtype == torch.int32
    assert trans.shape == (0, 1) and cover.shape == (0, 1)
    np.testing.assert_array_equal(color.cpu().numpy(), ref["color"])
    np.testing.assert_array_equal(allmap.cpu().numpy(), ref["others"])
    # shape_dims wider than L*F: the extra channels are zero (C2F buffer layout)
    hs2 = hs._replace(shape_dims=torch.tensor([0, sp.C + 8, sp.C + 8], dtype=torch.int32))
    color2, *_ = GaussianRasterizer(rs, hs2)(means3D=t(sc.means), means2D=None, opacities=t(sc.opacity),
                                             shs=torch.zeros(1, device=DEV), scales=t(sc.scales),
                                             rotations=t(sc.rotations), homotrans=t(sc.homotrans),
                                             ap_level=t(sc.ap_level), features=t(sc.table), offsets=t(sc.offsets),
                                             gridrange=t(np.asarray(sp.gridrange, np.float32)))
    c2 = color2.cpu().numpy()
    np.testing.assert_array_equal(c2[:sp.C], ref["color"])
    assert not c2[sp.C:].any()
    # coarse-to-fine: fewer active levels zero the later channels
    hs3 = hs._replace(L=3)
    color3, *_ = GaussianRasterizer(rs, hs3)(means3D=t(sc.means), means2D=None, opacities=t(sc.opacity),
                                             shs=torch.zeros(1, device=DEV), scales=t(sc.scales),
                                             rotations=t(sc.rotations), homotrans=t(sc.homotrans),
                                             ap_level=t(sc.ap_level), features=t(sc.table), offsets=t(sc.offsets),
                                             gridrange=t(np.asarray(sp.gridrange, np.float32)))
    c3 = color3.cpu().numpy()
    np.testing.assert_array_equal(c3[:3 * sp.F], ref["color"][:3 * sp.F])
    assert not c3[3 * sp.F:].any()


def test_colour_path_level0(oracle):
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("cfg1")
    sp = sc.spec
    cam = sc.cameras[0]
    rng = np.random.default_rng(1)
    cols = rng.uniform(0, 1, (sp.P, 3)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, cam.world_view_transform,
                                       cam.full_proj_transform, 0, cam.camera_center, False, False, 0.0, False, False)
    hs = HashGridSettings(0, 0.0, 0, False, 0, torch.empty(0))
    color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(means3D=t(sc.means), means2D=None, opacities=t(sc.opacity),
                                                           colors_precomp=t(cols), scales=t(sc.scales),
                                                           rotations=t(sc.rotations))
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    r = oracle.render(pre, b, W, H, 3, None, colors=cols)
    np.testing.assert_array_equal(color.cpu().numpy(), r["color"])
    np.testing.assert_array_equal(allmap.cpu().numpy()[:8], r["others"][:8])


def test_rvq_scene_end_to_end(oracle):
    """Decode RVQ attributes on the GPU (bit-exact), then render with them."""
    from nest_splat.rvq import RVQAttributes
    from nest_splat.scene import RVQ_BIAS
    from nest_splat import rasterizer as rz
    sc = scene("rvq_small")
    sp = sc.spec
    rv = RVQAttributes.from_numpy(sc.rvq_codebooks, sc.rvq_indices, RVQ_BIAS, DEV)
    dec = rv.decode()
    raw = {a: oracle.rvq_decode(sc.rvq_codebooks[a], sc.rvq_indices[a], RVQ_BIAS[a]) for a in RVQ_BIAS}
    scales, rots, op = oracle.activate(raw["scale"], raw["rotation"], raw["opacity"])
    np.testing.assert_array_equal(dec["scale"].cpu().numpy(), scales)
    np.testing.assert_array_equal(dec["rotation"].cpu().numpy(), rots)
    np.testing.assert_array_equal(dec["opacity"].cpu().numpy()[:, 0], op)
    from nest_splat.scene import build_homotrans_np
    homo = build_homotrans_np(rots, scales, sc.means)
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32))
    res = rz.rasterize_forward(settings, grid, t(sc.means), dec["opacity"], dec["scale"], dec["rotation"],
                               homotrans=t(homo), ap_level=t(sc.ap_level), channels=sp.C)
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, scales, rots, op, cam.world_view_transform, cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, sp.C, g, homotrans=homo, ap_level=sc.ap_level)
    assert res.num_rendered == b["num_rendered"]
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


def test_unsupported_modes_raise():
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("cfg1")
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, cam.world_view_transform,
                                       cam.full_proj_transform, 0, cam.camera_center, False, False, 0.0, False, False)
    hs = HashGridSettings(0, 0.0, 0, False, 0, torch.empty(0))
    kw = dict(means3D=t(sc.means), means2D=None, opacities=t(sc.opacity), colors_precomp=t(sc.means),
              scales=t(sc.scales), rotations=t(sc.rotations))
    for mode in (11, 15, 4 | 0x100):
        with pytest.raises(NotImplementedError):
            GaussianRasterizer(rs, hs)(render_mode=mode, **kw)
    with pytest.raises(NotImplementedError):
        GaussianRasterizer(rs, hs)(kernel_type=4, **kw)
    with pytest.raises(ValueError):
        GaussianRasterizer(rs, hs)(kernel_type=1, **kw)  # the beta kernel needs shapes
    with pytest.raises(Exception):
        GaussianRasterizer(rs, hs)(means3D=t(sc.means), means2D=None, opacities=t(sc.opacity))
    with pytest.raises(ValueError):
        GaussianRasterizer(rs, hs)(**{**kw, "means3D": t(sc.means[:, :2])})


def test_empty_and_culled_scenes():
    from nest_splat import rasterizer as rz
    sc = scene("cfg1")
    sp = sc.spec
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32))
    e = torch.zeros((0, 3), device=DEV)
    res = rz.rasterize_forward(settings, grid, e, torch.zeros((0, 1), device=DEV), torch.zeros((0, 2), device=DEV),
                               torch.zeros((0, 4), device=DEV), homotrans=torch.zeros((0, 4, 4), device=DEV),
                               channels=sp.C)
    assert res.num_rendered == 0 and not res.color.any()
    assert (res.others[1] == 0).all()
    # every splat behind the camera: all culled, nothing rendered
    forward = np.asarray(cam.world_view_transform[:3, 2], np.float32)  # camera z axis in world space
    behind = (sc.means - 1000.0 * forward[None, :]).astype(np.float32)
    res = rz.rasterize_forward(settings, grid, t(behind), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               homotrans=t(sc.homotrans), channels=sp.C)
    assert res.num_rendered == 0 and int(res.radii.abs().sum()) == 0 and not res.color.any()
