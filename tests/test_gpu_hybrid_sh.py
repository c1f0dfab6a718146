"""GPU parity of the hybrid SH render modes 8 (hybrid_SH), 9 (hybrid_SH_post)
and 10 (hybrid_SH_raw) (CR/forward.cu:1378-1542) against the oracle, bit for
bit: one 3-channel float32 grid level (hashed, as the reference builds it at
the finest resolution, and dense), rows of 3 raw colours or 48 SH
coefficients, every decompose setting, the contracted unbounded scene, with
the transmittance record and a kernel type.  The drop-in GaussianRasterizer
decodes the reference's packed level into the same call."""
import numpy as np
import pytest
import torch

from nest_splat.scene import get_spec, make_scene

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# (name, base spec, overrides): a hashed finest-resolution level (the
# reference's hybrid SH grid), a dense one, and the contracted 1M-splat layout
SCENES = {
    "shell_hashed": ("cfg2", dict(P=20_000, W=256, H=192, L=1, F=3, log2T=16, base_res=512)),
    "cube_dense": ("cfg1", dict(L=1, F=3, log2T=14, base_res=16)),
    "unbounded_hashed": ("cfg3", dict(P=60_000, W=320, H=216, L=1, F=3, log2T=17, base_res=2048)),
}
_cache = {}


def _scene(name):
    if name not in _cache:
        base, kw = SCENES[name]
        _cache[name] = make_scene(get_spec(base, name=f"hsh_{name}", **kw))
    return _cache[name]


def _rows(sc, mode, seed=3):
    rng = np.random.default_rng(seed)
    return rng.normal(0.0, 1.0 if mode != 9 else 0.5, (sc.spec.P, 48 if mode == 9 else 3)).astype(np.float32)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def run_gpu(sc, mode, dec, rows, C, record=False, kernel_type=0, shapes=None, levels=1):
    from nest_splat import rasterizer as rz
    sp = sc.spec
    cam = sc.cameras[0]
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                cam.world_view_transform, cam.full_proj_transform, cam.camera_center,
                                if_contract=sp.contract)
    grid = rz.HashGridDesc(levels, 3, sp.S, sp.base_res, _t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32),
                           render_mode=mode, decompose=dec)
    res = rz.rasterize_forward(settings, grid, _t(sc.means), _t(sc.opacity), _t(sc.scales), _t(sc.rotations),
                               homotrans=_t(sc.homotrans), ap_level=_t(sc.ap_level), colors_precomp=_t(rows), channels=C,
                               record_transmittance=record, kernel_type=kernel_type,
                               shapes=None if shapes is None else _t(shapes))
    torch.cuda.synchronize()
    return res


def run_oracle(O, sc, mode, dec, rows, C, record=False, kernel_type=0, shapes=None, levels=1):
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    pre = O.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                       cam.full_proj_transform, W, H)
    b = O.binning(pre, W, H)
    grid = O.make_grid(1, 3, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = O.render(pre, b, W, H, C, grid, homotrans=sc.homotrans, ap_level=sc.ap_level, colors=rows, render_mode=mode,
                 level=(dec << 24) | (3 << 16) | (levels << 8), record_transmittance=record, kernel_type=kernel_type,
                 shapes=shapes)
    return b, r


def _check(res, b, r):
    from nest_splat import rasterizer as rz
    W, H = r["color"].shape[2], r["color"].shape[1]
    assert res.num_rendered == b["num_rendered"]
    ba = {k: v.cpu().numpy() for k, v in rz.binning_arrays(res, W, H).items()}
    np.testing.assert_array_equal(ba["n_contrib"].view(np.uint32), r["n_contrib"])
    np.testing.assert_array_equal(ba["final_T"], r["final_T"])
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    color = res.color.cpu().numpy()
    assert np.abs(r["color"]).max() > 0
    np.testing.assert_array_equal(color, r["color"])


@pytest.mark.parametrize("name", list(SCENES))
@pytest.mark.parametrize("mode", [8, 9, 10])
@pytest.mark.parametrize("dec", [0, 1, 2])
def test_hybrid_sh_parity(oracle, name, mode, dec):
    sc = _scene(name)
    C = 48 if mode == 9 else 3
    print(f"[case] hybrid SH mode {mode} decompose {dec} {name}", flush=True)
    rows = _rows(sc, mode)
    _check(run_gpu(sc, mode, dec, rows, C), *run_oracle(oracle, sc, mode, dec, rows, C))


def test_hybrid_sh_extra_channels_record_and_kernel_type(oracle):
    """Mode 8 into 8 output channels (the 5 past the mode's stay 0), with the
    transmittance record and the general kernel; mode 10 without grid levels."""
    sc = _scene("shell_hashed")
    rows = _rows(sc, 8)
    shapes = np.random.default_rng(4).uniform(2.0, 6.0, sc.spec.P).astype(np.float32)
    print("[case] hybrid SH mode 8, C=8, record, kernel_type 3", flush=True)
    res = run_gpu(sc, 8, 0, rows, 8, record=True, kernel_type=3, shapes=shapes)
    b, r = run_oracle(oracle, sc, 8, 0, rows, 8, record=True, kernel_type=3, shapes=shapes)
    _check(res, b, r)
    assert not res.color[3:].any()
    np.testing.assert_array_equal(res.cover_pixels.cpu().numpy().reshape(-1), r["cover_pixels"])
    print("[case] hybrid SH mode 10 without grid levels", flush=True)
    _check(run_gpu(sc, 10, 0, rows, 3, levels=0), *run_oracle(oracle, sc, 10, 0, rows, 3, levels=0))


def test_hybrid_sh_through_drop_in(oracle):
    """GaussianRasterizer with render_mode 8 / 9 and the reference's packed
    level (decompose << 24 | SH degree << 16 | 1 << 8, GR:617-626) matches
    the direct call."""
    import math
    from diff_surfel_rasterization import GaussianRasterizationSettings, GaussianRasterizer, HashGridSettings
    sc = _scene("shell_hashed")
    sp = sc.spec
    cam = sc.cameras[0]
    for mode, dec in ((8, 0), (9, 2)):
        C = 48 if mode == 9 else 3
        rows = _rows(sc, mode)
        print(f"[case] drop-in hybrid SH mode {mode} decompose {dec}", flush=True)
        rs = GaussianRasterizationSettings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                           torch.zeros(3, device=DEV), 1.0, _t(cam.world_view_transform),
                                           _t(cam.full_proj_transform), 3, _t(cam.camera_center), False, False, 0.0,
                                           sp.contract, False)
        hs = HashGridSettings((dec << 24) | (3 << 16) | (1 << 8), math.log2(sp.per_level_scale), sp.base_res, False, 0,
                              torch.tensor([0, C, C], dtype=torch.int32))
        color, radii, allmap, _, _ = GaussianRasterizer(rs, hs)(
            means3D=_t(sc.means), means2D=None, opacities=_t(sc.opacity), colors_precomp=_t(rows),
            scales=_t(sc.scales), rotations=_t(sc.rotations), homotrans=_t(sc.homotrans), ap_level=_t(sc.ap_level),
            features=_t(sc.table), offsets=_t(sc.offsets), gridrange=_t(np.asarray(sp.gridrange, np.float32)),
            render_mode=mode)
        res = run_gpu(sc, mode, dec, rows, C)
        np.testing.assert_array_equal(color.cpu().numpy(), res.color.cpu().numpy())
        np.testing.assert_array_equal(allmap.cpu().numpy(), res.others.cpu().numpy())
