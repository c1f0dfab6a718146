"""GPU parity of the backward pass (nest_backward, nest_grid_encode_backward)
against the backward oracle, which the CPU tests pin against float64
autograd.  The forward state both sides start from is the GPU forward, which
is bit-exact with the oracle's.  The reference sums every per-splat and
per-table-entry gradient with float atomics in hardware order; here the GPU
sums per wave then atomically, the oracle sequentially, so the comparison is
relative to each gradient array's largest entry: max |gpu - oracle| <= 2e-5
* max |oracle| (float32 reassociation of sums of up to a few thousand terms).
"""
import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-5


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _shapes(kt, P, seed):
    """Per-splat kernel parameters: beta-kernel shapes 0.2-4, flex betas 0-2
    (every 7th 0), general exponents 2-8 (every 9th below 2)."""
    rng = np.random.default_rng(seed)
    if kt == 1:
        return rng.uniform(0.2, 4.0, P).astype(np.float32)
    if kt == 2:
        v = rng.uniform(0.0, 2.0, P).astype(np.float32)
        v[::7] = 0.0
        return v
    v = rng.uniform(2.0, 8.0, P).astype(np.float32)
    v[::9] = rng.uniform(0.8, 2.0, v[::9].shape).astype(np.float32)
    return v


def _setup(oracle, sc, path, beta=0.0, sh_degree=3, kt=0):
    from nest_splat import rasterizer as rz
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, beta=beta, if_contract=sp.contract)
    rng = np.random.default_rng(17)
    P = sp.P
    kw = dict(homotrans=None, ap_level=None, colors_precomp=None, shs=None, sh_degree=0)
    shapes = None
    if kt:
        shapes = _shapes(kt, P, 70 + kt)
        kw.update(shapes=_t(shapes), kernel_type=kt)
    if path == "hash":
        C = sp.C
        grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, _t(sc.table), sc.offsets,
                               np.asarray(sp.gridrange, np.float32))
        ap = sc.ap_level.reshape(-1).copy()
        ap[::5] = 3.0
        kw.update(homotrans=_t(sc.homotrans), ap_level=_t(ap))
    else:
        grid = rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
        if path == "colors":
            C = 8
            colors = rng.uniform(0, 1, (P, C)).astype(np.float32)
            kw.update(colors_precomp=_t(colors))
        else:
            C = 3
            shs = (rng.standard_normal((P, 16, 3)) * 0.8).astype(np.float32)
            kw.update(shs=_t(shs), sh_degree=sh_degree)
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               channels=C, **kw)
    dcol = rng.standard_normal((C, H, W)).astype(np.float32)
    doth = rng.standard_normal((14, H, W)).astype(np.float32)
    gb = rz.rasterize_backward(settings, grid, res, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               _t(dcol), _t(doth), channels=C, **kw)
    torch.cuda.synchronize()
    gpu = {k: (None if v is None else v.cpu().numpy()) for k, v in vars(gb).items()}

    # oracle on the same forward state
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    campos = np.asarray(cam.camera_center, np.float32)
    if path == "hash":
        g = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
        fwd = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=ap, beta=beta, kernel_type=kt,
                            shapes=shapes)
        ob = oracle.render_backward(pre, b, fwd, W, H, C, g, dcol, doth, homotrans=sc.homotrans.reshape(-1, 16),
                                    ap_level=ap, beta=beta, kernel_type=kt, shapes=shapes)
        pb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"],
                                        cam.world_view_transform, cam.full_proj_transform, W, H, ob["dtransmat"],
                                        ob["dhomo"], ob["dnormal"], ob["dmean2D"])
    else:
        if path == "colors":
            cols, extra = colors, {}
        else:
            cols, clamped = oracle.sh_colors(pre, sc.means, campos, shs, sh_degree)
            extra = dict(shs=shs, sh_degree=sh_degree, campos=campos, clamped=clamped)
        fwd = oracle.render(pre, b, W, H, C, None, colors=cols, beta=beta, kernel_type=kt, shapes=shapes)
        ob = oracle.render_backward(pre, b, fwd, W, H, C, None, dcol, doth, colors=cols, beta=beta, kernel_type=kt,
                                    shapes=shapes)
        pb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"],
                                        cam.world_view_transform, cam.full_proj_transform, W, H, ob["dtransmat"],
                                        ob["dhomo"], ob["dnormal"], ob["dmean2D"], dcolors=ob["dcolors"], **extra)
    np.testing.assert_array_equal(res.color.cpu().numpy(), fwd["color"])  # same forward state
    ref = dict(dmeans3D=pb["dmeans"], dmeans2D=pb["dmean2D"], dopacity=ob["dopacity"][:, None],
               dscales=pb["dscales"], drotations=pb["drots"])
    if path == "hash":
        ref["dfeatures"] = ob["dtable"].reshape(gpu["dfeatures"].shape)
        ref["dgradsum"] = ob["gradsum"][:, None]
    else:
        ref["dcolors"] = ob["dcolors"]
        if path == "sh":
            ref["dshs"] = pb["dshs"]
    if kt:
        ref["dshapes"] = ob["dshapes"]
    return gpu, ref, pre


def _compare(gpu, ref, pre):
    vis = pre["radii"] > 0
    for k, r in ref.items():
        o = gpu[k]
        assert o.shape == r.shape, (k, o.shape, r.shape)
        assert np.isfinite(o).all(), k
        assert np.abs(r).max() > 0, k
        err = _rel(o, r)
        print(f"{k}: max rel err {err:.2e}", flush=True)
        assert err < TOL, (k, err)
        if k not in ("dfeatures",):
            assert not o[~vis].any(), k  # culled splats get no gradient


@pytest.mark.parametrize("name", ["cfg1", "shell_small", "unbounded_small", "unbounded_f8", "unbounded_f1"])
def test_backward_hash_parity(oracle, name):
    sc = scene(name)
    print(f"[case] backward hash {name} P={sc.spec.P}", flush=True)
    _compare(*_setup(oracle, sc, "hash"))


@pytest.mark.parametrize("path,beta", [("colors", 0.0), ("sh", 0.0), ("colors", 1.5)])
def test_backward_colour_parity(oracle, path, beta):
    sc = scene("shell_small")
    print(f"[case] backward {path} beta={beta}", flush=True)
    _compare(*_setup(oracle, sc, path, beta=beta))


def test_backward_hash_beta_parity(oracle):
    sc = scene("cfg1")
    print("[case] backward hash beta=0.8", flush=True)
    _compare(*_setup(oracle, sc, "hash", beta=0.8))


@pytest.mark.parametrize("name,path,kt,beta", [("cfg1", "hash", 1, 0.0), ("unbounded_small", "hash", 3, 0.0),
                                               ("shell_small", "hash", 2, 0.8), ("shell_small", "colors", 1, 0.0),
                                               ("shell_small", "colors", 2, 1.5), ("shell_small", "sh", 3, 0.0)])
def test_backward_kernel_types_parity(oracle, name, path, kt, beta):
    """kernel_type 1 (beta), 2 (flex) and 3 (general) (CR/backward.cu:764-803,
    :1864-1909, :1963-2039): every gradient and dL/dshape against the
    oracle."""
    sc = scene(name)
    print(f"[case] backward kernel_type {kt} {path} {name} beta={beta}", flush=True)
    _compare(*_setup(oracle, sc, path, beta=beta, kt=kt))


@pytest.mark.parametrize("interp,align", [(0, False), (1, True)])
def test_grid_encode_backward_parity(oracle, interp, align):
    from gridencoder import GridEncoder
    rng = np.random.default_rng(3 + interp)
    enc = GridEncoder(3, 8, 2, 1.5, 16, 14, align_corners=align,
                      interpolation="smoothstep" if interp else "linear").to(DEV)
    with torch.no_grad():
        enc.embeddings.copy_(torch.from_numpy(rng.standard_normal(tuple(enc.embeddings.shape)).astype(np.float32) * 0.2))
    B = 5000
    x = rng.uniform(-0.02, 1.02, (B, 3)).astype(np.float32)
    xt = _t(x).requires_grad_(True)
    y = enc(xt)
    g = rng.standard_normal(tuple(y.shape)).astype(np.float32)
    y.backward(_t(g))
    torch.cuda.synchronize()
    tab = enc.embeddings.detach().cpu().numpy()
    grid = oracle.make_grid(8, 2, float(np.log2(1.5)), 16, enc._offsets_host, tab, (0.0, 1.0), False,
                            align_corners=align, interp=interp)
    gt, gi = oracle.grid_encode_backward(grid, x, g)
    e_t = _rel(enc.embeddings.grad.cpu().numpy(), gt)
    e_i = _rel(xt.grad.cpu().numpy(), gi)
    print(f"grid encode backward: table {e_t:.2e} inputs {e_i:.2e}")
    assert np.abs(gi).max() > 0 and np.abs(gt).max() > 0
    assert e_t < TOL and e_i < TOL
    oob = ((x < 0) | (x > 1)).any(1)
    assert oob.any() and not xt.grad.cpu().numpy()[oob].any()


def test_autograd_through_drop_in_rasterizer():
    """GaussianRasterizer forward + loss.backward() (the reference's training
    call, DSRpy:174-275) lands the same gradients in .grad as a direct
    nest_backward call, in the reference's slots (means2D gets the
    densification statistic, ap_level the |grad| sum)."""
    import math
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    from nest_splat import rasterizer as rz
    sc = scene("cfg1")
    sp = sc.spec
    cam = sc.cameras[0]
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, _t(cam.world_view_transform),
                                       _t(cam.full_proj_transform), 3, _t(cam.camera_center), False, False, 0.0,
                                       sp.contract, False)
    hs = HashGridSettings(sp.L, math.log2(sp.per_level_scale), sp.base_res, False, 0,
                          torch.tensor([0, sp.C, sp.C], dtype=torch.int32, device=DEV))
    leaf = lambda a: _t(a).requires_grad_(True)
    means, means2D = leaf(sc.means), torch.zeros(sp.P, 3, device=DEV, requires_grad=True)
    opac, scales, rots = leaf(sc.opacity), leaf(sc.scales), leaf(sc.rotations)
    table, ap = leaf(sc.table), leaf(sc.ap_level)
    color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(
        means3D=means, means2D=means2D, opacities=opac, shs=torch.zeros(sp.P, 16, 3, device=DEV), scales=scales,
        rotations=rots, homotrans=_t(sc.homotrans), ap_level=ap, features=table, offsets=_t(sc.offsets),
        gridrange=_t(np.asarray(sp.gridrange, np.float32)))
    rng = np.random.default_rng(23)
    dcol = _t(rng.standard_normal(tuple(color.shape)).astype(np.float32))
    doth = _t(rng.standard_normal(tuple(allmap.shape)).astype(np.float32))
    ((color * dcol).sum() + (allmap * doth).sum()).backward()
    torch.cuda.synchronize()

    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, _t(sc.table), sc.offsets,
                           np.asarray(sp.gridrange, np.float32))
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               homotrans=_t(sc.homotrans), ap_level=_t(sc.ap_level), channels=sp.C)
    gb = rz.rasterize_backward(settings, grid, res, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               dcol, doth, homotrans=_t(sc.homotrans), ap_level=_t(sc.ap_level), channels=sp.C)
    torch.cuda.synchronize()
    pairs = [(means.grad, gb.dmeans3D), (means2D.grad, gb.dmeans2D), (opac.grad, gb.dopacity),
             (scales.grad, gb.dscales), (rots.grad, gb.drotations), (table.grad, gb.dfeatures),
             (ap.grad, gb.dgradsum)]
    for got, ref in pairs:
        assert got is not None and tuple(got.shape) == tuple(ref.shape)
        err = _rel(got.cpu().numpy(), ref.cpu().numpy())
        assert err < 1e-5, err


def test_autograd_kernel_type_through_drop_in_rasterizer():
    """kernel_type 3 through the drop-in: shapes.grad is the [P, 1] dL/dshape
    of a direct nest_backward call (DSRpy:241-271 returns grad_shapes in the
    shapes slot)."""
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    from nest_splat import rasterizer as rz
    sc = scene("shell_small")
    sp = sc.spec
    cam = sc.cameras[0]
    rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                       torch.zeros(3, device=DEV), 1.0, _t(cam.world_view_transform),
                                       _t(cam.full_proj_transform), 0, _t(cam.camera_center), False, False, 0.0,
                                       sp.contract, False)
    hs = HashGridSettings(0, 0.0, 0, False, 0, torch.tensor([0, 3, 3], dtype=torch.int32, device=DEV))
    rng = np.random.default_rng(29)
    cols = rng.uniform(0, 1, (sp.P, 3)).astype(np.float32)
    shp = _shapes(3, sp.P, 91).reshape(-1, 1)
    leaf = lambda a: _t(a).requires_grad_(True)
    means, opac, scales, rots = leaf(sc.means), leaf(sc.opacity), leaf(sc.scales), leaf(sc.rotations)
    shapes = leaf(shp)
    color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(
        means3D=means, means2D=torch.zeros(sp.P, 3, device=DEV), opacities=opac, colors_precomp=_t(cols),
        scales=scales, rotations=rots, shapes=shapes, kernel_type=3)
    dcol = _t(rng.standard_normal(tuple(color.shape)).astype(np.float32))
    doth = _t(rng.standard_normal(tuple(allmap.shape)).astype(np.float32))
    ((color * dcol).sum() + (allmap * doth).sum()).backward()
    torch.cuda.synchronize()

    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
    kw = dict(colors_precomp=_t(cols), channels=3, shapes=_t(shp.reshape(-1)), kernel_type=3)
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations), **kw)
    gb = rz.rasterize_backward(settings, grid, res, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               dcol, doth, **kw)
    torch.cuda.synchronize()
    assert tuple(shapes.grad.shape) == (sp.P, 1)
    assert np.abs(gb.dshapes.cpu().numpy()).max() > 0
    for got, ref in [(shapes.grad.reshape(-1), gb.dshapes), (means.grad, gb.dmeans3D), (opac.grad, gb.dopacity),
                     (scales.grad, gb.dscales), (rots.grad, gb.drotations)]:
        err = _rel(got.cpu().numpy(), ref.cpu().numpy())
        assert err < 1e-5, err
