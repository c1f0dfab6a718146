"""GPU parity of the dual-grid render modes 2 (baseline_double) and 3
(baseline_blend_double) (CR/forward.cu:1146-1217, :1975-2004) against the
oracle, bit for bit: a second grid at the splat centres (its own table,
offsets and range), affine and contracted scenes, float32 and binary16 first
grids, splats querying fewer levels, with and without the second grid, and
through the drop-in GaussianRasterizer with features_diffuse."""
import math

import numpy as np
import pytest
import torch

from nest_splat.scene import get_spec, make_scene

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

SCENES = {
    "shell": ("cfg2", dict(P=20_000, W=256, H=192, L=6, F=4, log2T=15)),
    "unbounded": ("cfg3", dict(P=60_000, W=320, H=216, L=8, F=4, log2T=16)),
    "shells_f16": ("cfg5", dict(P=40_000, W=240, H=136, L=8, F=4, log2T=15, n_cams=1)),
}
_cache = {}


def _scene(name):
    if name not in _cache:
        base, kw = SCENES[name]
        sc = make_scene(get_spec(base, name=f"dual_{name}", **kw))
        rng = np.random.default_rng(31)
        table2 = rng.uniform(-0.2, 0.2, (sc.table.shape[0], 4)).astype(np.float32)
        range2 = np.float32([sc.spec.gridrange[0] * 1.1, sc.spec.gridrange[1] * 0.95])
        ap = sc.ap_level.reshape(-1, 1).copy()
        ap[::5] = 3.0
        _cache[name] = (sc, table2, range2, ap)
    return _cache[name]


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def run_gpu(sc, table2, range2, ap, mode, second=True, record=False):
    from nest_splat import rasterizer as rz
    sp = sc.spec
    cam = sc.cameras[0]
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                cam.world_view_transform, cam.full_proj_transform, cam.camera_center,
                                if_contract=sp.contract)
    grid = rz.HashGridDesc(sp.L, 4, sp.S, sp.base_res, _t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32),
                           render_mode=mode, table2=_t(table2) if second else None,
                           offsets2=sc.offsets if second else None, gridrange2=range2 if second else None)
    C = (2 if mode == 2 else 1) * sp.L * 4
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               homotrans=_t(sc.homotrans), ap_level=_t(ap), channels=C, record_transmittance=record)
    torch.cuda.synchronize()
    return res


def run_oracle(O, sc, table2, range2, ap, mode, second=True, record=False):
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    pre = O.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                       cam.full_proj_transform, W, H)
    b = O.binning(pre, W, H)
    grid = O.make_grid(sp.L, 4, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    C = (2 if mode == 2 else 1) * sp.L * 4
    r = O.render(pre, b, W, H, C, grid, homotrans=sc.homotrans, ap_level=ap, render_mode=mode, level=sp.L,
                 grid2=(sc.offsets, table2, range2) if second else None, record_transmittance=record)
    return b, r


def _check(res, b, r):
    from nest_splat import rasterizer as rz
    W, H = r["color"].shape[2], r["color"].shape[1]
    assert res.num_rendered == b["num_rendered"]
    ba = {k: v.cpu().numpy() for k, v in rz.binning_arrays(res, W, H).items()}
    np.testing.assert_array_equal(ba["n_contrib"].view(np.uint32), r["n_contrib"])
    np.testing.assert_array_equal(ba["final_T"], r["final_T"])
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    assert np.abs(r["color"]).max() > 0
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


@pytest.mark.parametrize("name", list(SCENES))
@pytest.mark.parametrize("mode", [2, 3])
def test_dual_grid_parity(oracle, name, mode):
    sc, table2, range2, ap = _scene(name)
    print(f"[case] dual grid mode {mode} {name}", flush=True)
    _check(run_gpu(sc, table2, range2, ap, mode), *run_oracle(oracle, sc, table2, range2, ap, mode))


@pytest.mark.parametrize("mode", [2, 3])
def test_dual_grid_without_second_grid_and_record(oracle, mode):
    sc, table2, range2, ap = _scene("shell")
    print(f"[case] dual grid mode {mode} without the second grid, record", flush=True)
    res = run_gpu(sc, table2, range2, ap, mode, second=False, record=True)
    b, r = run_oracle(oracle, sc, table2, range2, ap, mode, second=False, record=True)
    _check(res, b, r)
    np.testing.assert_array_equal(res.cover_pixels.cpu().numpy().reshape(-1), r["cover_pixels"])


def test_dual_grid_through_drop_in(oracle):
    """GaussianRasterizer(render_mode=2 / 3, features_diffuse=...) equals the
    direct call (GR's diffuse grid arguments, DSRpy:277-396)."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc, table2, range2, ap = _scene("unbounded")
    sp = sc.spec
    cam = sc.cameras[0]
    for mode in (2, 3):
        print(f"[case] drop-in dual grid mode {mode}", flush=True)
        C = (2 if mode == 2 else 1) * sp.L * 4
        rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                           torch.zeros(3, device=DEV), 1.0, _t(cam.world_view_transform),
                                           _t(cam.full_proj_transform), 3, _t(cam.camera_center), False, False, 0.0,
                                           sp.contract, False)
        hs = HashGridSettings(sp.L, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                              torch.tensor([0, C, C], dtype=torch.int32))
        color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(
            means3D=_t(sc.means), means2D=None, opacities=_t(sc.opacity), shs=torch.zeros(sp.P, 16, 3, device=DEV),
            scales=_t(sc.scales),
            rotations=_t(sc.rotations), homotrans=_t(sc.homotrans), ap_level=_t(ap), features=_t(sc.table),
            offsets=_t(sc.offsets), gridrange=_t(np.asarray(sp.gridrange, np.float32)), features_diffuse=_t(table2),
            offsets_diffuse=_t(sc.offsets), gridrange_diffuse=_t(range2), render_mode=mode)
        res = run_gpu(sc, table2, range2, ap, mode)
        np.testing.assert_array_equal(color.cpu().numpy(), res.color.cpu().numpy())
        np.testing.assert_array_equal(allmap.cpu().numpy(), res.others.cpu().numpy())


SURF = {
    # (base spec, overrides, mode): 12 features per level (mode 1, with and without the
    # second grid) and 15 (mode 5), affine and contracted
    "shell_m1": ("cfg2", dict(P=20_000, W=256, H=192, L=6, F=12, log2T=14), 1),
    "unbounded_m1": ("cfg3", dict(P=40_000, W=256, H=160, L=16, F=12, log2T=13), 1),
    "shell_m5": ("cfg2", dict(P=20_000, W=256, H=192, L=6, F=15, log2T=14), 5),
    "unbounded_m5": ("cfg3", dict(P=40_000, W=256, H=160, L=9, F=15, log2T=13), 5),
}


@pytest.mark.parametrize("name", list(SURF))
@pytest.mark.parametrize("second", [True, False])
def test_surface_modes_parity(oracle, name, second):
    """Render modes 1 and 5 (CR/forward.cu:1825-1908) bit for bit against the
    oracle: the potentials dotted with the splat normal per hit, the centre
    features (mode 1: the second grid; mode 5: the grid's colours)."""
    from nest_splat import rasterizer as rz
    base, kw, mode = SURF[name]
    sc = make_scene(get_spec(base, name=f"surf_{name}", **kw))
    sp = sc.spec
    rng = np.random.default_rng(41)
    table2 = rng.uniform(-0.1, 0.1, ((1 << sp.log2T) * sp.L, 4)).astype(np.float32)
    range2 = np.float32([sp.gridrange[0] * 1.05, sp.gridrange[1] * 0.9])
    ap = sc.ap_level.reshape(-1, 1).copy()
    ap[::6] = 2.0
    C = (4 if mode == 1 else 7) * sp.L
    print(f"[case] surface mode {mode} {name} second={second}", flush=True)
    cam = sc.cameras[0]
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                cam.world_view_transform, cam.full_proj_transform, cam.camera_center,
                                if_contract=sp.contract)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, _t(sc.table), sc.offsets,
                           np.asarray(sp.gridrange, np.float32), render_mode=mode,
                           table2=_t(table2) if second else None, offsets2=sc.offsets if second else None,
                           gridrange2=range2 if second else None)
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               homotrans=_t(sc.homotrans), ap_level=_t(ap), channels=C)
    torch.cuda.synchronize()
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    og = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, C, og, homotrans=sc.homotrans, ap_level=ap, render_mode=mode, level=sp.L,
                      grid2=(sc.offsets, table2, range2) if second else None)
    _check(res, b, r)


@pytest.mark.parametrize("mode", [1, 2, 3, 5, 8, 9, 10])
def test_new_modes_on_empty_and_culled_scenes(mode):
    """No splats, and every splat behind the camera: nothing rendered, zeros
    out, in each of the inline-lookup and centre-feature modes."""
    from nest_splat import rasterizer as rz
    F = {1: 12, 5: 15, 8: 3, 9: 3, 10: 3}.get(mode, 4)
    L = 1 if mode in (8, 9, 10) else 3
    sc = make_scene(get_spec("cfg1", L=L, F=F, log2T=10, name=f"empty_{mode}"))
    sp = sc.spec
    cam = sc.cameras[0]
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform)
    grid = rz.HashGridDesc(L, F, sp.S, sp.base_res, _t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32),
                           render_mode=mode)
    C = {1: 4 * L, 2: 8 * L, 3: 4 * L, 5: 7 * L, 8: 3, 9: 48, 10: 3}[mode]
    width = {8: 3, 9: 48, 10: 3}.get(mode)
    print(f"[case] empty scene, mode {mode}", flush=True)
    z = lambda *s: torch.zeros(s, device=DEV)
    res = rz.rasterize_forward(settings, grid, z(0, 3), z(0, 1), z(0, 2), z(0, 4), homotrans=z(0, 4, 4),
                               ap_level=z(0, 1), colors_precomp=z(0, width) if width else None, channels=C)
    torch.cuda.synchronize()
    assert res.num_rendered == 0 and not res.color.any() and not res.others.any()
    forward = np.asarray(cam.world_view_transform[:3, 2], np.float32)
    behind = (sc.means - 1000.0 * forward[None, :]).astype(np.float32)
    rows = torch.ones((sp.P, width), device=DEV) if width else None
    res = rz.rasterize_forward(settings, grid, _t(behind), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               homotrans=_t(sc.homotrans), ap_level=_t(sc.ap_level), colors_precomp=rows, channels=C)
    torch.cuda.synchronize()
    assert res.num_rendered == 0 and not res.color.any()
