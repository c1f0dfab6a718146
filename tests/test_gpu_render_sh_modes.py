"""render()'s SH-rasterised appearance modes (gaussian_renderer/__init__.py:88-114,
:686-692, :799-903): ``diffuse`` and ``specular`` rasterise SH colours,
``diffuse_ngp`` adds the hash grid's MLP colour at the back-projected median
depth, ``diffuse_offset`` queries the grid at that point moved by the rendered
colour - 0.5 (clamped to +-0.1) or, with use_xyz_mode, at the blended splat
centres (allmap 8:11).

Each is checked against the same composition of oracle stages on the CPU:
SH colours, preprocess, binning and render, the back-projection in float32
numpy, the grid encode and the MLP.  The rasterised image is bit-exact; the
grid colour allows 5e-4 (measured: 4.5e-5 at most; the binary16 MLP, and an
ulp of the query point from the GPU's matrix product, which the trilinear
interpolation turns into a change of the same order).
"""
import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
NGP_TOL = 5e-4


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _sh(P, seed=7):
    return np.random.default_rng(seed).normal(0, 0.5, (P, 16, 3)).astype(np.float32)


def _expected(oracle, sc, shs, mode, use_xyz, bg):
    from nest_splat.camera import view_ray_matrix
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    deg = 3 if mode == "specular" else 0
    cols, _ = oracle.sh_colors(pre, sc.means, np.asarray(cam.camera_center, np.float32), shs, deg)
    r = oracle.render(pre, b, W, H, 3, None, colors=cols)
    img = r["color"].copy()
    alpha = r["others"][1]
    ngp = None
    if mode in ("diffuse_ngp", "diffuse_offset"):
        gx, gy = np.meshgrid(np.arange(W, dtype=np.float32), np.arange(H, dtype=np.float32), indexing="xy")
        pix = np.stack([gx, gy, np.ones_like(gx)], -1).reshape(-1, 3)
        rays_d = pix @ view_ray_matrix(cam)
        c2w = np.linalg.inv(cam.world_view_transform.astype(np.float64).T).astype(np.float32)
        med = np.nan_to_num(r["others"][5]).reshape(-1, 1)
        if mode == "diffuse_offset" and use_xyz:
            base = r["others"][8:11].reshape(3, -1).T
        else:
            base = med * rays_d + c2w[:3, 3]
        if mode == "diffuse_offset":
            base = base + np.clip(img.reshape(3, -1).T - np.float32(0.5), -0.1, 0.1)
        vmin, vmax = np.float32(sp.gridrange[0]), np.float32(sp.gridrange[1])
        x = (base - vmin) / (vmax - vmin)
        grid = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, False)
        feat = oracle.grid_encode(grid, x.astype(np.float32))
        dirs = rays_d / np.linalg.norm(rays_d, axis=1, keepdims=True)
        ngp = oracle.mlp(feat.T.copy(), dirs.astype(np.float32), alpha.reshape(-1), sc.W1, sc.W2, sc.W3,
                         sp.mlp_dtype).reshape(3, H, W)
    return img, alpha, ngp


@pytest.mark.parametrize("mode,use_xyz", [("diffuse", False), ("specular", False), ("diffuse_ngp", False),
                                          ("diffuse_offset", False), ("diffuse_offset", True)])
def test_sh_modes_against_oracle(oracle, mode, use_xyz):
    from nest_splat.renderer import Pipe, SplatModel, render, scene_to_device
    sc = scene("shell_small")
    sp = sc.spec
    assert not sp.contract
    print(f"[case] render mode {mode} use_xyz={use_xyz}", flush=True)
    shs = _sh(sp.P)
    _, ingp = scene_to_device(sc, "cuda:0")
    pc = SplatModel(_t(sc.means), _t(sc.scales), _t(sc.rotations), _t(sc.opacity), _t(sc.ap_level),
                    homotrans=_t(sc.homotrans), features=_t(shs), active_sh_degree=3)
    bg = np.float32([0.2, 0.1, 0.3])
    out = render(sc.cameras[0], pc, Pipe(), _t(bg), ingp=ingp, mode=mode, use_xyz_mode=use_xyz)
    torch.cuda.synchronize()
    img, alpha, ngp = _expected(oracle, sc, shs, mode, use_xyz, bg)
    got = out["render"].cpu().numpy()
    bgmap = (np.float32(1) - alpha)[None] * bg[:, None, None]
    if ngp is None:
        np.testing.assert_array_equal(got, img + bgmap)
        return
    gn = out["ngp_rgb"].cpu().numpy()
    assert (alpha > 0).mean() > 0.2 and np.abs(ngp).max() > 0.1
    err = np.abs(gn - ngp)
    print(f"ngp colour: max err {err.max():.2e}, mean {err.mean():.2e}", flush=True)
    assert err.max() < NGP_TOL and err.mean() < 1e-4
    assert not gn[:, alpha == 0].any()  # masked where nothing was hit
    if mode == "diffuse_ngp":
        np.testing.assert_array_equal(out["gaussian_rgb"].cpu().numpy(), img)
        np.testing.assert_allclose(got, img + gn + bgmap, rtol=0, atol=1e-6)
    else:
        np.testing.assert_array_equal(out["gaussian_rgb"].cpu().numpy(), img - np.float32(0.5))
        np.testing.assert_allclose(got, gn + bgmap, rtol=0, atol=1e-6)
        if use_xyz:
            sl = out["scout_loss_data"]
            assert tuple(sl["points_base"].shape) == (sp.W * sp.H, 3)
