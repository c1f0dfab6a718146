"""Scenes loaded from disk render on the GPU bit for bit like the oracle on
the same loaded attributes: a splat PLY (SH colour path, and hash path with
the loaded appearance level 6) and an ngp_<iter>.pth hash grid."""
import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _write_scene(tmp_path, sc, seed=0):
    """Raw parameters of a synthetic scene written as the reference writes them."""
    from nest_splat import model_io as M
    rng = np.random.default_rng(seed)
    P = sc.spec.P
    raw = M.RawSplats(sc.means.astype(np.float32), rng.normal(0, 0.6, (P, 1, 3)).astype(np.float32),
                      rng.normal(0, 0.3, (P, 15, 3)).astype(np.float32),
                      np.log(sc.opacity / (1 - sc.opacity)).reshape(P, 1).astype(np.float32),
                      np.log(sc.scales).astype(np.float32), sc.rotations.astype(np.float32))
    ply = str(tmp_path / "point_cloud.ply")
    M.save_splats_ply(ply, raw)
    ngp = str(tmp_path / "ngp_30000.pth")
    M.save_ngp(ngp, sc.table, sc.offsets)
    return ply, ngp


def test_loaded_ply_renders_like_oracle(oracle, tmp_path):
    from nest_splat import model_io as M
    from nest_splat import rasterizer as rz
    from nest_splat.scene import build_homotrans_np
    sc = scene("cfg1")
    sp = sc.spec
    cam = sc.cameras[0]
    ply, ngp = _write_scene(tmp_path, sc)
    raw = M.load_splats_ply(ply)
    a = raw.activated()
    shs = raw.shs()
    W, H = cam.image_width, cam.image_height
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, if_contract=sp.contract)
    pre = oracle.preprocess(a["xyz"], a["scales"], a["rotations"], a["opacity"], cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    print("[case] loaded PLY, SH colour path", flush=True)
    grid0 = rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
    res = rz.rasterize_forward(settings, grid0, _t(a["xyz"]), _t(a["opacity"]), _t(a["scales"]), _t(a["rotations"]),
                               channels=3, shs=_t(shs), sh_degree=raw.sh_degree)
    rgb, _ = oracle.sh_colors(pre, a["xyz"], np.asarray(cam.camera_center, np.float32), shs, raw.sh_degree)
    r = oracle.render(pre, b, W, H, 3, None, colors=rgb)
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])
    print("[case] loaded PLY + ngp, hash path at ap_level 6", flush=True)
    ck = M.load_ngp(ngp)
    np.testing.assert_array_equal(ck.embeddings, sc.table)
    homo = build_homotrans_np(a["rotations"], a["scales"], a["xyz"])
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, _t(ck.embeddings), ck.offsets,
                           np.asarray(sp.gridrange, np.float32))
    res = rz.rasterize_forward(settings, grid, _t(a["xyz"]), _t(a["opacity"]), _t(a["scales"]), _t(a["rotations"]),
                               homotrans=_t(homo), ap_level=_t(a["ap_level"]), channels=sp.C)
    g = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, ck.offsets.astype(np.int32), ck.embeddings, sp.gridrange,
                         sp.contract)
    r = oracle.render(pre, b, W, H, sp.C, g, homotrans=homo, ap_level=a["ap_level"])
    col = res.color.cpu().numpy()
    np.testing.assert_array_equal(col, r["color"])
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    # levels 6 and 7 are past the loaded appearance level: no features there
    assert sp.L > 6 and not col[6 * sp.F:].any() and col[:6 * sp.F].any()
