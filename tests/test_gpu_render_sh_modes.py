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


@pytest.mark.parametrize("mode,dec", [("hybrid_SH", None), ("hybrid_SH_raw", "ngp_only"),
                                      ("hybrid_SH_post", None), ("hybrid_SH_post", "gaussian_only")])
def test_hybrid_modes_against_oracle(oracle, mode, dec):
    """render()'s hybrid SH branches (GR:600-680, :958-1000) against the oracle's
    render modes 8-10 fed with the same rows (raw SH colours from eval_sh, which
    the CPU tests pin, or the 48 coefficients), the mask, and for hybrid_SH_post
    the per-pixel SH colour along the view ray."""
    from gridencoder import GridEncoder
    from nest_splat.renderer import DECOMPOSE, HYBRID_MODES, HashINGP, Pipe, SplatModel, eval_sh, render
    from nest_splat.scene import get_spec, make_scene
    sc = make_scene(get_spec("cfg2", P=20_000, W=256, H=192, L=1, F=3, log2T=16, base_res=512, name="hsh_render"))
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    print(f"[case] render {mode} decompose {dec}", flush=True)
    shs = _sh(sp.P, seed=11)
    enc = GridEncoder(3, 1, 3, 1.0, sp.base_res, sp.log2T).to(DEV)
    assert enc.offsets.cpu().numpy().tolist() == [int(v) for v in sc.offsets]
    with torch.no_grad():
        enc.embeddings = torch.nn.Parameter(_t(sc.table), requires_grad=False)
    ingp = HashINGP(enc, None, sp.gridrange, sp.contract)
    pc = SplatModel(_t(sc.means), _t(sc.scales), _t(sc.rotations), _t(sc.opacity), _t(sc.ap_level),
                    homotrans=_t(sc.homotrans), features=_t(shs), active_sh_degree=3)
    bg = np.float32([0.2, 0.1, 0.3])
    out = render(cam, pc, Pipe(), _t(bg), ingp=ingp, mode=mode, decompose_mode=dec, with_surface=False)
    torch.cuda.synchronize()

    rmode = HYBRID_MODES[mode]
    shs_view = torch.from_numpy(shs).transpose(1, 2)
    if rmode == 9:
        rows = shs_view.reshape(-1, 48).numpy()
    else:
        d = torch.from_numpy(sc.means) - torch.from_numpy(np.asarray(cam.camera_center, np.float32))
        rows = eval_sh(3, shs_view, d / d.norm(dim=1, keepdim=True)).numpy()
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    grid = oracle.make_grid(1, 3, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, 48 if rmode == 9 else 3, grid, homotrans=sc.homotrans, ap_level=sc.ap_level,
                      colors=np.ascontiguousarray(rows, np.float32), render_mode=rmode,
                      level=(DECOMPOSE[dec] << 24) | (3 << 16) | (1 << 8))
    alpha = r["others"][1]
    mask = (alpha > 0).astype(np.float32)
    if rmode == 9:
        coeffs = torch.from_numpy(r["color"].reshape(48, -1).T.copy()).reshape(-1, 3, 16)
        dirs = torch.from_numpy(oracle.ray_dirs(cam))
        img = torch.clamp_min(eval_sh(3, coeffs, dirs) + 0.5, 0.0).numpy().T.reshape(3, H, W) * mask
    else:
        img = r["color"] * mask
    img = img + (np.float32(1) - alpha)[None] * bg[:, None, None]
    got = out["render"].cpu().numpy()
    err = np.abs(got - img).max()
    print(f"render {mode}: max err {err:.2e}", flush=True)
    assert np.abs(img).max() > 0.1 and err < 1e-5
