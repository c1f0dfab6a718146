"""GPU parity of render modes 4 (cat), 6 (adaptive), 7 (adaptive_add), 12 (adaptive_cat),
13 (adaptive_cat_fast) and 14 (adaptive_zero), training and inference, against the oracle, bit for bit, on the shared small scenes:
per-splat feature rows ahead of a grid of the scene's first levels, with
f32 and f16 tables, level_dim 2 and 4, the common-grid lookup and the
general per-level one (smoothstep), mixed fast/slow splats in inference.
The drop-in GaussianRasterizer decodes the reference's packed L into the
same call."""
import math

import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _rows(sc, width, weight_col=None, seed=0):
    rng = np.random.default_rng(seed)
    rows = rng.uniform(-1, 1, (sc.spec.P, width)).astype(np.float32)
    if weight_col is not None:
        rows[:, weight_col] = rng.uniform(0, 1, sc.spec.P).astype(np.float32)
    return rows


def run_gpu(sc, render_mode, hyb, glevels, total, C, rows, interp=0, record=False):
    from nest_splat import rasterizer as rz
    sp = sc.spec
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                cam.world_view_transform, cam.full_proj_transform, cam.camera_center,
                                if_contract=sp.contract)
    grid = rz.HashGridDesc(glevels, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets,
                           np.asarray(sp.gridrange, np.float32), interpolation=interp, render_mode=render_mode,
                           hybrid_levels=hyb, total_levels=total)
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), colors_precomp=t(rows), channels=C,
                               record_transmittance=record)
    torch.cuda.synchronize()
    return res


def run_oracle(O, sc, render_mode, level, grid_levels, C, rows, interp=0, record=False):
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    pre = O.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                       cam.full_proj_transform, W, H)
    b = O.binning(pre, W, H)
    grid = O.make_grid(grid_levels, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract,
                       interp=interp)
    r = O.render(pre, b, W, H, C, grid, homotrans=sc.homotrans, ap_level=sc.ap_level, colors=rows,
                 render_mode=render_mode, level=level, record_transmittance=record)
    return b, r


def _check(res, b, r):
    from nest_splat import rasterizer as rz
    sc_W, sc_H = r["color"].shape[2], r["color"].shape[1]
    assert res.num_rendered == b["num_rendered"]
    ba = {k: v.cpu().numpy() for k, v in rz.binning_arrays(res, sc_W, sc_H).items()}
    np.testing.assert_array_equal(ba["n_contrib"].view(np.uint32), r["n_contrib"])
    np.testing.assert_array_equal(ba["final_T"], r["final_T"])
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    color = res.color.cpu().numpy()
    scale = max(np.abs(r["color"]).max(), 1e-30)
    np.testing.assert_allclose(color, r["color"], rtol=1e-5, atol=1e-5 * scale)
    np.testing.assert_array_equal(color, r["color"])


# (scene, per-splat levels, grid levels, extra zero channels): level_dim 4
# f32 (contracted) and f16, level_dim 2; 32- and 64-channel accumulators
CAT_CASES = [("unbounded_small", 4, 10, 0), ("shells_small", 2, 5, 4), ("shell_small", 6, 16, 0),
             ("shell_small", 0, 9, 2)]


@pytest.mark.parametrize("name,hyb,gl,extra", CAT_CASES)
def test_cat_mode_parity(oracle, name, hyb, gl, extra):
    sc = scene(name)
    F = sc.spec.F
    C = (hyb + gl) * F + extra
    print(f"[case] mode 4 {name} hyb={hyb} grid levels={gl} C={C}", flush=True)
    rows = _rows(sc, hyb * F, seed=hyb)
    res = run_gpu(sc, 4, hyb, gl, 0, C, rows)
    # the oracle counts the grid levels from the offsets, as the reference
    b, r = run_oracle(oracle, sc, 4, ((hyb + gl) << 16) | (1 << 8) | hyb, gl, C, rows)
    _check(res, b, r)


# (scene, inference, total levels, per-splat levels, active grid levels, interp)
ACF_CASES = [("unbounded_small", True, 16, 10, 4, 0), ("shells_small", False, 8, 5, 3, 0),
             ("shell_small", True, 12, 4, 8, 1), ("unbounded_small", False, 6, 1, 5, 1),
             ("shells_small", True, 16, 12, 0, 0)]


@pytest.mark.parametrize("name,infer,total,hyb,hl,interp", ACF_CASES)
def test_adaptive_cat_fast_parity(oracle, name, infer, total, hyb, hl, interp):
    sc = scene(name)
    F = sc.spec.F
    tdim = total * F
    mode = 13 | (0x100 if infer else 0)
    print(f"[case] mode {mode:#x} {name} total={total} hyb={hyb} hl={hl} interp={interp}", flush=True)
    rows = _rows(sc, tdim + 1, weight_col=tdim, seed=total + hyb)
    res = run_gpu(sc, mode, hyb, hl, total, tdim, rows, interp=interp)
    b, r = run_oracle(oracle, sc, mode, (total << 16) | (hl << 8) | hyb, max(hl, 1), tdim, rows, interp=interp)
    _check(res, b, r)
    if infer:
        assert not r["n_contrib"][0].any()


# (scene, total levels, grid levels, interp); f32 and f16 tables
AA_CASES = [("unbounded_small", 16, 6, 0), ("shells_small", 8, 5, 0), ("shell_small", 12, 8, 1), ("cfg1", 8, 8, 0)]


@pytest.mark.parametrize("name,total,hl,interp", AA_CASES)
def test_adaptive_add_parity(oracle, name, total, hl, interp):
    """Render mode 7 (adaptive_add): every channel weight * row + (1 - weight)
    * grid, the grid zero past its levels; full hits."""
    sc = scene(name)
    tdim = total * sc.spec.F
    print(f"[case] mode 7 {name} total={total} hl={hl} interp={interp}", flush=True)
    rows = _rows(sc, tdim + 1, weight_col=tdim, seed=total + hl + 3)
    res = run_gpu(sc, 7, 0, hl, total, tdim, rows, interp=interp)
    b, r = run_oracle(oracle, sc, 7, (total << 16) | (hl << 8), max(hl, 1), tdim, rows, interp=interp)
    _check(res, b, r)


# (scene, grid levels, extra channels, interp): level_dim 4 f32 (contracted,
# 64 channels) and f16, level_dim 2; rows wider than the blended channels
AD_CASES = [("unbounded_small", 16, 0, 0), ("shells_small", 5, 3, 0), ("shell_small", 8, 4, 1), ("cfg1", 6, 2, 0),
            ("cfg1", 3, 9, 1)]


@pytest.mark.parametrize("name,levels,extra,interp", AD_CASES)
def test_adaptive_parity(oracle, name, levels, extra, interp):
    """Render mode 6 (adaptive): rows of C floats, the first levels*F channels
    0.5 * row + 0.5 * grid, the rest 0; full hits."""
    sc = scene(name)
    C = levels * sc.spec.F + extra
    print(f"[case] mode 6 {name} levels={levels} C={C} interp={interp}", flush=True)
    rows = _rows(sc, C, seed=levels + extra)
    res = run_gpu(sc, 6, 0, levels, 0, C, rows, interp=interp)
    b, r = run_oracle(oracle, sc, 6, levels, levels, C, rows, interp=interp)
    _check(res, b, r)
    if extra:
        assert not res.color[levels * sc.spec.F:].any()


def test_adaptive_record_and_kernel_type(oracle):
    """Render mode 6 with the transmittance record and the general kernel
    (kernel_type 3), against the oracle, bit for bit."""
    from nest_splat import rasterizer as rz
    sc = scene("shell_small")
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    levels = 6
    C = levels * sp.F + 2
    rows = _rows(sc, C, seed=61)
    shapes = np.random.default_rng(62).uniform(2.0, 7.0, sp.P).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    print("[case] mode 6 shell_small, record, kernel_type 3", flush=True)
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(levels, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets,
                           np.asarray(sp.gridrange, np.float32), render_mode=6)
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), colors_precomp=t(rows), channels=C,
                               record_transmittance=True, kernel_type=3, shapes=t(shapes))
    torch.cuda.synchronize()
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(levels, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=sc.ap_level, colors=rows, render_mode=6,
                      level=levels, record_transmittance=True, kernel_type=3, shapes=shapes)
    _check(res, b, r)
    np.testing.assert_array_equal(res.cover_pixels.cpu().numpy().reshape(-1), r["cover_pixels"])
    # transmittance sums land by atomics in any order: float sums within 1e-5
    scale = max(float(np.abs(r["trans_avg"]).max()), 1e-30)
    np.testing.assert_allclose(res.trans_avg.cpu().numpy().reshape(-1), r["trans_avg"], rtol=1e-5, atol=1e-6 * scale)
    assert r["cover_pixels"].any()


# (scene, inference, total levels, per-splat levels, grid levels, interp)
AZ_CASES = [("unbounded_small", False, 16, 10, 6, 0), ("shells_small", True, 9, 5, 3, 0),
            ("shell_small", True, 12, 4, 8, 1), ("cfg1", False, 8, 3, 5, 1)]


@pytest.mark.parametrize("name,infer,total,hyb,hl,interp", AZ_CASES)
def test_adaptive_zero_parity(oracle, name, infer, total, hyb, hl, interp):
    """Render mode 14 (adaptive_zero): coarse rows, then the grid times the
    weight; weights <= 1e-6 (training) or < 0.1 (inference) skip the grid."""
    sc = scene(name)
    F = sc.spec.F
    pgd = hyb * F
    mode = 14 | (0x100 if infer else 0)
    print(f"[case] mode {mode:#x} {name} total={total} hyb={hyb} hl={hl} interp={interp}", flush=True)
    rows = _rows(sc, pgd + 1, weight_col=pgd, seed=total + hyb + 2)
    rows[::11, pgd] = 0.0
    res = run_gpu(sc, mode, hyb, hl, total, total * F, rows, interp=interp)
    b, r = run_oracle(oracle, sc, mode, (total << 16) | (hl << 8) | hyb, max(hl, 1), total * F, rows, interp=interp)
    _check(res, b, r)


# (scene, inference, total levels, per-splat levels, active grid levels, interp)
AC_CASES = [("unbounded_small", False, 16, 10, 6, 0), ("shells_small", True, 8, 5, 3, 0),
            ("shell_small", True, 12, 4, 8, 1), ("cfg1", False, 8, 3, 5, 1)]


@pytest.mark.parametrize("name,infer,total,hyb,hl,interp", AC_CASES)
def test_adaptive_cat_parity(oracle, name, infer, total, hyb, hl, interp):
    """Render mode 12 (adaptive_cat): unweighted coarse rows, blended (training)
    or weight >= 0.9 fast (inference) grid levels, full hits."""
    sc = scene(name)
    F = sc.spec.F
    tdim = total * F
    mode = 12 | (0x100 if infer else 0)
    print(f"[case] mode {mode:#x} {name} total={total} hyb={hyb} hl={hl} interp={interp}", flush=True)
    rows = _rows(sc, tdim + 1, weight_col=tdim, seed=total + hyb + 1)
    res = run_gpu(sc, mode, hyb, hl, total, tdim, rows, interp=interp)
    b, r = run_oracle(oracle, sc, mode, (total << 16) | (hl << 8) | hyb, max(hl, 1), tdim, rows, interp=interp)
    _check(res, b, r)
    assert r["n_contrib"][0].any()


def test_drop_in_decodes_packed_levels(oracle):
    """GaussianRasterizer with render_mode 4 / 13 | 0x100 and the packed L of
    the reference's render() (GR:224-226, :395-396)."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("shells_small")
    sp = sc.spec
    cam = sc.cameras[0]
    F = sp.F
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, t(cam.world_view_transform),
                                       t(cam.full_proj_transform), 3, t(cam.camera_center), False, False, 0.0,
                                       sp.contract, False)
    for mode, total, hyb, gl in ((4, 8, 3, 5), (13 | 0x100, 10, 6, 3), (6, 7, 0, 7)):
        C = total * F
        width = hyb * F if mode == 4 else (C if mode == 6 else C + 1)
        rows = _rows(sc, width, weight_col=None if mode in (4, 6) else C, seed=mode)
        offs = np.zeros(17, np.int32)
        offs[:gl + 1] = np.asarray(sc.offsets)[:gl + 1]
        # mode 6 takes L as the grid's level count
        packed = gl if mode == 6 else (total << 16) | ((1 if mode == 4 else gl) << 8) | hyb
        hs = HashGridSettings(packed, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                              torch.tensor([hyb * F, gl * F, C], dtype=torch.int32, device=DEV))
        print(f"[case] drop-in mode {mode:#x} L={packed:#x}", flush=True)
        color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(
            means3D=t(sc.means), means2D=None, opacities=t(sc.opacity), colors_precomp=t(rows),
            scales=t(sc.scales), rotations=t(sc.rotations), homotrans=t(sc.homotrans), ap_level=t(sc.ap_level),
            features=t(sc.table), offsets=t(offs), gridrange=t(np.asarray(sp.gridrange, np.float32)),
            render_mode=mode)
        torch.cuda.synchronize()
        _, r = run_oracle(oracle, sc, mode, packed, gl, C, rows)
        np.testing.assert_array_equal(allmap.cpu().numpy(), r["others"])
        np.testing.assert_array_equal(color.cpu().numpy(), r["color"])


# (mode, scene, total levels, per-splat levels, grid levels): training and
# inference; mode 13 records nothing
REC_CASES = [(4, "unbounded_small", 0, 4, 10), (12, "shell_small", 12, 4, 8), (12 | 0x100, "shells_small", 8, 5, 3),
             (13, "unbounded_small", 16, 10, 6), (14, "cfg1", 8, 3, 5), (7, "shell_small", 10, 0, 6)]


@pytest.mark.parametrize("mode,name,total,hyb,gl", REC_CASES)
def test_record_transmittance_modes(oracle, mode, name, total, hyb, gl):
    """record_transmittance in the mixed modes: every hit that reaches the
    blend records (CR/forward.cu:1961-1964), mode 13's hits leave the loop
    first (:1090)."""
    sc = scene(name)
    F = sc.spec.F
    base = mode & 0xFF
    print(f"[case] record_transmittance mode {mode:#x} {name}", flush=True)
    if base == 4:
        C = (hyb + gl) * F
        rows = _rows(sc, hyb * F, seed=hyb)
        res = run_gpu(sc, 4, hyb, gl, 0, C, rows, record=True)
        b, r = run_oracle(oracle, sc, 4, ((hyb + gl) << 16) | (1 << 8) | hyb, gl, C, rows, record=True)
    elif base == 14:
        rows = _rows(sc, hyb * F + 1, weight_col=hyb * F, seed=total + hyb + 2)
        rows[::11, hyb * F] = 0.0
        res = run_gpu(sc, mode, hyb, gl, total, total * F, rows, record=True)
        b, r = run_oracle(oracle, sc, mode, (total << 16) | (gl << 8) | hyb, max(gl, 1), total * F, rows, record=True)
    elif base == 7:
        rows = _rows(sc, total * F + 1, weight_col=total * F, seed=total + gl + 3)
        res = run_gpu(sc, 7, 0, gl, total, total * F, rows, record=True)
        b, r = run_oracle(oracle, sc, 7, (total << 16) | (gl << 8), max(gl, 1), total * F, rows, record=True)
    else:
        rows = _rows(sc, total * F + 1, weight_col=total * F, seed=total + hyb)
        res = run_gpu(sc, mode, hyb, gl, total, total * F, rows, record=True)
        b, r = run_oracle(oracle, sc, mode, (total << 16) | (gl << 8) | hyb, max(gl, 1), total * F, rows,
                          record=True)
    _check(res, b, r)
    cover = res.cover_pixels.cpu().numpy()
    np.testing.assert_array_equal(cover, r["cover_pixels"])
    scale = max(float(np.abs(r["trans_avg"]).max()), 1e-30)
    np.testing.assert_allclose(res.trans_avg.cpu().numpy(), r["trans_avg"], rtol=1e-5, atol=1e-6 * scale)
    if base == 13:
        assert not cover.any() and r["others"][7].any()
    else:
        assert cover.sum() == r["others"][7].sum() > 0


def test_drop_in_record_transmittance(oracle):
    """GaussianRasterizer with record_transmittance=True returns the
    reference's (transmittance_avg, cover_pixels) as [P, 1] tensors."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("shell_small")
    sp = sc.spec
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, t(cam.world_view_transform),
                                       t(cam.full_proj_transform), 3, t(cam.camera_center), False, False, 0.0,
                                       sp.contract, True)
    hs = HashGridSettings(sp.L, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                          torch.tensor([0, 0, sp.L * sp.F], dtype=torch.int32, device=DEV))
    print("[case] drop-in record_transmittance", flush=True)
    out = GaussianRasterizer(rs, hs)(
        means3D=t(sc.means), means2D=None, opacities=t(sc.opacity), scales=t(sc.scales), rotations=t(sc.rotations),
        colors_precomp=torch.zeros((sp.P, sp.L * sp.F), device=DEV), homotrans=t(sc.homotrans),
        ap_level=t(sc.ap_level), features=t(sc.table), offsets=t(np.asarray(sc.offsets)),
        gridrange=t(np.asarray(sp.gridrange, np.float32)))
    torch.cuda.synchronize()
    trans, cover = out[3], out[4]
    assert trans.shape == (sp.P, 1) and cover.shape == (sp.P, 1)
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    grid = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, sp.L * sp.F, grid, homotrans=sc.homotrans, ap_level=sc.ap_level,
                      record_transmittance=True)
    np.testing.assert_array_equal(cover.cpu().numpy()[:, 0], r["cover_pixels"])
    scale = max(float(np.abs(r["trans_avg"]).max()), 1e-30)
    np.testing.assert_allclose(trans.cpu().numpy()[:, 0], r["trans_avg"], rtol=1e-5, atol=1e-6 * scale)


def test_mode_validation():
    """Mode arguments the library rejects before any launch."""
    from nest_splat import rasterizer as rz
    sc = scene("cfg1")  # level_dim 2
    sp = sc.spec
    cam = sc.cameras[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                cam.world_view_transform, cam.full_proj_transform, cam.camera_center)

    def call(mode, hyb, gl, total, C, width):
        grid = rz.HashGridDesc(gl, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets,
                               np.asarray(sp.gridrange, np.float32), render_mode=mode, hybrid_levels=hyb,
                               total_levels=total)
        rows = t(np.zeros((sp.P, width), np.float32))
        return rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                                    homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), colors_precomp=rows,
                                    channels=C)

    errs = (NotImplementedError, RuntimeError)
    with pytest.raises(errs, match="render_mode 11"):
        call(11, 1, 2, 4, 8, 8)
    with pytest.raises(errs, match="supported"):
        call(4 | 0x100, 1, 2, 0, 8, 2)
    with pytest.raises(errs, match="exceed total_levels"):
        call(13, 3, 3, 5, 10, 11)
    with pytest.raises(errs, match="channels"):
        call(4, 2, 4, 0, 10, 4)
    with pytest.raises(errs, match="<= 32"):
        call(13, 1, 2, 40, 80, 81)
    with pytest.raises(errs, match="hybrid_levels must be 0"):
        call(7, 1, 2, 4, 8, 9)
    with pytest.raises(errs, match="hybrid_levels must be 0"):
        call(6, 1, 2, 0, 8, 8)
    with pytest.raises(errs, match="channels"):
        call(6, 0, 4, 0, 6, 6)
    # modes without a backward in the reference: 13, the inference flag and 6
    for mode in (13, 12 | 0x100, 14 | 0x100, 6):
        grid = rz.HashGridDesc(2, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets,
                               np.asarray(sp.gridrange, np.float32), render_mode=mode,
                               hybrid_levels=0 if mode == 6 else 1, total_levels=4)
        rows = t(np.zeros((sp.P, grid.row_width(8)), np.float32))
        kw = dict(homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), colors_precomp=rows, channels=8)
        res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations), **kw)
        with pytest.raises(errs, match="forward-only"):
            rz.rasterize_backward(settings, grid, res, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                                  None, None, **kw)


# (scene, per-splat levels, grid levels, active grid levels): level_dim 2 and
# 4 (contracted); all levels active, coarse-to-fine (fewer active than
# rendered) and none active (rows only)
CAT_BWD_CASES = [("cfg1", 2, 6, 6), ("shell_small", 4, 12, 7), ("unbounded_small", 4, 10, 10), ("cfg1", 3, 5, 0)]


@pytest.mark.parametrize("name,hyb,gl,active", CAT_BWD_CASES)
def test_cat_mode_backward_parity(oracle, name, hyb, gl, active):
    """nest_backward in render mode 4 against the backward oracle (which the
    CPU tests pin against float64 autograd), on the same forward state.  The
    sums run in another order on each side (per wave then atomically on the
    GPU, sequentially in the oracle): 2e-5 of each array's largest entry."""
    from nest_splat import rasterizer as rz
    sc = scene(name)
    sp = sc.spec
    F = sp.F
    pgd = hyb * F
    C = (hyb + gl) * F
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    print(f"[case] mode 4 backward {name} hyb={hyb} grid levels={gl} active={active}", flush=True)
    rows = _rows(sc, pgd, seed=hyb + 40)
    ap = sc.ap_level.reshape(-1).copy()
    ap[::5] = 3.0
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(gl, F, sp.S, sp.base_res, t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32),
                           render_mode=4, hybrid_levels=hyb, active_levels=active)
    kw = dict(homotrans=t(sc.homotrans), ap_level=t(ap), colors_precomp=t(rows), channels=C)
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations), **kw)
    rng = np.random.default_rng(23)
    dcol = rng.standard_normal((C, H, W)).astype(np.float32)
    doth = rng.standard_normal((14, H, W)).astype(np.float32)
    gb = rz.rasterize_backward(settings, grid, res, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               t(dcol), t(doth), **kw)
    torch.cuda.synchronize()
    gpu = {k: (None if v is None else v.cpu().numpy()) for k, v in vars(gb).items()}

    level = ((hyb + gl) << 16) | (active << 8) | hyb
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(gl, F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    fwd = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=ap, colors=rows, render_mode=4,
                        level=level)
    np.testing.assert_array_equal(res.color.cpu().numpy(), fwd["color"])  # same forward state
    ob = oracle.render_backward(pre, b, fwd, W, H, C, g, dcol, doth, homotrans=sc.homotrans.reshape(-1, 16),
                                ap_level=ap, colors=rows, render_mode=4, level=level)
    pb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"],
                                    cam.world_view_transform, cam.full_proj_transform, W, H, ob["dtransmat"],
                                    ob["dhomo"], ob["dnormal"], ob["dmean2D"])
    ref = dict(dmeans3D=pb["dmeans"], dmeans2D=pb["dmean2D"], dopacity=ob["dopacity"][:, None],
               dscales=pb["dscales"], drotations=pb["drots"], dcolors=ob["dcolors"], dgradsum=ob["gradsum"][:, None],
               dfeatures=ob["dtable"].reshape(gpu["dfeatures"].shape))
    vis = pre["radii"] > 0
    for k, r in ref.items():
        o = gpu[k]
        assert o.shape == r.shape, (k, o.shape, r.shape)
        assert np.isfinite(o).all(), k
        if k == "dfeatures" and active == 0:
            assert not o.any() and not r.any()
            continue
        assert np.abs(r).max() > 0, k
        err = float(np.abs(o.astype(np.float64) - r).max() / np.abs(r).max())
        print(f"{k}: max rel err {err:.2e}", flush=True)
        assert err < 2e-5, (k, err)
        if k != "dfeatures":
            assert not o[~vis].any(), k
    if 0 < active < gl:  # the levels past the active ones get no gradient
        assert not gpu["dfeatures"].reshape(-1)[int(sc.offsets[active]) * F:].any()


def test_drop_in_cat_modes_autograd(oracle):
    """GaussianRasterizer in render mode 4 under autograd, with the
    reference's packed L (7 of 12 grid levels active): the gradients of the
    per-splat rows, the table and the means reach the leaves and match the
    oracle; mode 12 gives the direct call's gradients; mode 13 has no
    backward and says so."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = scene("shell_small")
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    F, hyb, gl, active = sp.F, 3, 12, 7
    pgd, C = hyb * F, (hyb + gl) * F
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    rs = GaussianRasterizationSettings(H, W, cam.tanfovx, cam.tanfovy, torch.zeros(3, device=DEV), 1.0,
                                       t(cam.world_view_transform), t(cam.full_proj_transform), 3,
                                       t(cam.camera_center), False, False, 0.0, sp.contract, False)
    offs = np.zeros(17, np.int32)
    offs[:gl + 1] = np.asarray(sc.offsets)[:gl + 1]
    packed = ((hyb + gl) << 16) | (active << 8) | hyb
    hs = HashGridSettings(packed, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                          torch.tensor([pgd, gl * F, C], dtype=torch.int32, device=DEV))
    rows = _rows(sc, pgd, seed=5)
    leaf = lambda a: t(a).requires_grad_(True)
    means, rows_t, table = leaf(sc.means), leaf(rows), leaf(sc.table)
    print(f"[case] drop-in mode 4 autograd L={packed:#x}", flush=True)
    color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(
        means3D=means, means2D=None, opacities=t(sc.opacity), colors_precomp=rows_t, scales=t(sc.scales),
        rotations=t(sc.rotations), homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), features=table,
        offsets=t(offs), gridrange=t(np.asarray(sp.gridrange, np.float32)), render_mode=4)
    rng = np.random.default_rng(29)
    dcol = rng.standard_normal((C, H, W)).astype(np.float32)
    doth = rng.standard_normal((14, H, W)).astype(np.float32)
    doth[7:] = 0  # channels 7-13 carry no gradient
    ((color * t(dcol)).sum() + (allmap * t(doth)).sum()).backward()
    torch.cuda.synchronize()

    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(gl, F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    fwd = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=sc.ap_level, colors=rows,
                        render_mode=4, level=packed)
    np.testing.assert_array_equal(color.detach().cpu().numpy(), fwd["color"])
    ob = oracle.render_backward(pre, b, fwd, W, H, C, g, dcol, doth, homotrans=sc.homotrans.reshape(-1, 16),
                                ap_level=sc.ap_level, colors=rows, render_mode=4, level=packed)
    pb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"],
                                    cam.world_view_transform, cam.full_proj_transform, W, H, ob["dtransmat"],
                                    ob["dhomo"], ob["dnormal"], ob["dmean2D"])
    for name, ours, ref in (("rows", rows_t.grad, ob["dcolors"]), ("table", table.grad, ob["dtable"]),
                            ("means3D", means.grad, pb["dmeans"])):
        o = ours.cpu().numpy().reshape(ref.shape).astype(np.float64)
        err = float(np.abs(o - ref).max() / np.abs(ref).max())
        print(f"{name}: max rel err {err:.2e}", flush=True)
        assert np.abs(ref).max() > 0 and err < 2e-5, (name, err)

    # mode 12 (adaptive_cat training) under autograd: the same gradients as
    # nest_backward called directly
    from nest_splat import rasterizer as rz
    packed12 = (8 << 16) | (3 << 8) | 2
    hs12 = HashGridSettings(packed12, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                            torch.tensor([0, 0, 8 * F], dtype=torch.int32, device=DEV))
    rows12 = _rows(sc, 8 * F + 1, weight_col=8 * F, seed=7)
    rows12_t, table12 = leaf(rows12), leaf(sc.table)
    color12, _, allmap12, _, _ = GaussianRasterizer(rs, hs12)(
        means3D=t(sc.means), means2D=None, opacities=t(sc.opacity), colors_precomp=rows12_t, scales=t(sc.scales),
        rotations=t(sc.rotations), homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), features=table12,
        offsets=t(offs), gridrange=t(np.asarray(sp.gridrange, np.float32)), render_mode=12)
    dcol12 = t(rng.standard_normal((8 * F, H, W)).astype(np.float32))
    ((color12 * dcol12).sum() + (allmap12 * t(doth)).sum()).backward()
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, if_contract=sp.contract)
    grid12 = rz.HashGridDesc(3, F, sp.S, sp.base_res, t(sc.table), offs.astype(np.int64),
                             np.asarray(sp.gridrange, np.float32), render_mode=12, hybrid_levels=2, total_levels=8)
    kw = dict(homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), colors_precomp=t(rows12), channels=8 * F)
    res12 = rz.rasterize_forward(settings, grid12, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations), **kw)
    gb12 = rz.rasterize_backward(settings, grid12, res12, t(sc.means), t(sc.opacity), t(sc.scales),
                                 t(sc.rotations), dcol12, t(doth), **kw)
    torch.cuda.synchronize()
    for name, ours, ref in (("rows12", rows12_t.grad, gb12.dcolors), ("table12", table12.grad, gb12.dfeatures)):
        o, r = ours.cpu().numpy().astype(np.float64), ref.cpu().numpy().reshape(ours.shape)
        assert np.abs(r).max() > 0 and np.abs(o - r).max() <= 2e-5 * np.abs(r).max(), name

    hs13 = HashGridSettings((8 << 16) | (3 << 8) | 2, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                            torch.tensor([0, 0, 8 * F], dtype=torch.int32, device=DEV))
    rows13 = leaf(_rows(sc, 8 * F + 1, weight_col=8 * F, seed=6))
    color13, _, _, _, _ = GaussianRasterizer(rs, hs13)(
        means3D=t(sc.means), means2D=None, opacities=t(sc.opacity), colors_precomp=rows13, scales=t(sc.scales),
        rotations=t(sc.rotations), homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), features=t(sc.table),
        offsets=t(offs), gridrange=t(np.asarray(sp.gridrange, np.float32)), render_mode=13)
    with pytest.raises(NotImplementedError, match="forward-only"):
        color13.sum().backward()


# (render mode, scene, total levels, per-splat levels, grid levels, kernel type)
AC_BWD_CASES = [(12, "cfg1", 8, 3, 5, 0), (12, "shell_small", 12, 4, 8, 0), (12, "unbounded_small", 16, 10, 6, 0),
                (12, "cfg1", 6, 2, 0, 0), (14, "cfg1", 8, 3, 5, 0), (14, "shell_small", 13, 4, 8, 0),
                (14, "unbounded_small", 16, 10, 6, 0), (7, "cfg1", 8, 0, 5, 0), (7, "unbounded_small", 16, 0, 6, 0),
                (12, "shell_small", 12, 4, 8, 1), (14, "cfg1", 8, 3, 5, 3), (7, "cfg1", 8, 0, 5, 2)]


def _kt_shapes(kt, P, seed):
    rng = np.random.default_rng(seed)
    if kt == 1:
        return rng.uniform(0.2, 4.0, P).astype(np.float32)
    if kt == 2:
        v = rng.uniform(0.0, 2.0, P).astype(np.float32)
        v[::7] = 0.0
        return v
    return rng.uniform(2.0, 8.0, P).astype(np.float32)


@pytest.mark.parametrize("mode,name,total,hyb,gl,kt", AC_BWD_CASES)
def test_adaptive_cat_backward_parity(oracle, mode, name, total, hyb, gl, kt):
    """nest_backward in render modes 7 (adaptive_add), 12 (adaptive_cat) and
    14 (adaptive_zero), training, against the backward oracle, which the CPU tests pin against
    float64 autograd: gradients of the rows and their blend weights, the
    table and the geometry, within 2e-5 of each array's largest entry.  Mode
    14 rows include weight-0 splats, whose grid levels are skipped.  Some
    cases use kernel types 1-3, with dL/dshape."""
    from nest_splat import rasterizer as rz
    sc = scene(name)
    sp = sc.spec
    F = sp.F
    tdim = total * F
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    print(f"[case] mode {mode} backward {name} total={total} hyb={hyb} grid levels={gl}", flush=True)
    nw = hyb * F if mode == 14 else tdim  # features ahead of the weight
    rows = _rows(sc, nw + 1, weight_col=nw, seed=total + 50)
    if mode == 14:
        rows[::9, nw] = 0.0
    ap = sc.ap_level.reshape(-1).copy()
    ap[::5] = 3.0
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(gl, F, sp.S, sp.base_res, t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32),
                           render_mode=mode, hybrid_levels=hyb, total_levels=total)
    kw = dict(homotrans=t(sc.homotrans), ap_level=t(ap), colors_precomp=t(rows), channels=tdim)
    shapes = None
    if kt:
        shapes = _kt_shapes(kt, sp.P, 60 + kt)
        kw.update(shapes=t(shapes), kernel_type=kt)
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations), **kw)
    rng = np.random.default_rng(31)
    dcol = rng.standard_normal((tdim, H, W)).astype(np.float32)
    doth = rng.standard_normal((14, H, W)).astype(np.float32)
    gb = rz.rasterize_backward(settings, grid, res, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               t(dcol), t(doth), **kw)
    torch.cuda.synchronize()
    gpu = {k: (None if v is None else v.cpu().numpy()) for k, v in vars(gb).items()}

    level = (total << 16) | (gl << 8) | hyb
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(max(gl, 1), F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    fwd = oracle.render(pre, b, W, H, tdim, g, homotrans=sc.homotrans, ap_level=ap, colors=rows, render_mode=mode,
                        level=level, kernel_type=kt, shapes=shapes)
    np.testing.assert_array_equal(res.color.cpu().numpy(), fwd["color"])  # same forward state
    ob = oracle.render_backward(pre, b, fwd, W, H, tdim, g, dcol, doth, homotrans=sc.homotrans.reshape(-1, 16),
                                ap_level=ap, colors=rows, render_mode=mode, level=level, kernel_type=kt,
                                shapes=shapes)
    pb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"],
                                    cam.world_view_transform, cam.full_proj_transform, W, H, ob["dtransmat"],
                                    ob["dhomo"], ob["dnormal"], ob["dmean2D"])
    ref = dict(dmeans3D=pb["dmeans"], dmeans2D=pb["dmean2D"], dopacity=ob["dopacity"][:, None],
               dscales=pb["dscales"], drotations=pb["drots"], drows=ob["dcolors"][:, :nw],
               dweight=ob["dcolors"][:, nw], dgradsum=ob["gradsum"][:, None])
    if kt:
        ref["dshapes"] = ob["dshapes"]
    gpu["drows"], gpu["dweight"] = gpu["dcolors"][:, :nw], gpu["dcolors"][:, nw]
    if gl > 0:
        ref["dfeatures"] = ob["dtable"].reshape(gpu["dfeatures"].shape)
    vis = pre["radii"] > 0
    for k, r in ref.items():
        o = gpu[k]
        assert o.shape == r.shape, (k, o.shape, r.shape)
        assert np.isfinite(o).all(), k
        if k == "dweight" and gl == 0:
            assert not o.any() and not r.any()
            continue
        assert np.abs(r).max() > 0, k
        err = float(np.abs(o.astype(np.float64) - r).max() / np.abs(r).max())
        print(f"{k}: max rel err {err:.2e}", flush=True)
        assert err < 2e-5, (k, err)
        if k != "dfeatures":
            assert not o[~vis].any(), k
