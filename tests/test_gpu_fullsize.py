"""Parity at the benchmark sizes: the 100k-splat 800x800 object scene (2^19
table, fp16 MLP, white background), the 500k-splat RVQ-compressed scene
(4096-entry codebooks decoded on the GPU, then rendered), the 1M-splat
1600x1064 unbounded scene and the 4M-splat 1920x1080 fp16-table scene (all
eight of its cameras).

The GPU renders the whole frame.  The oracle computes preprocess for every
splat and the render of every k-th tile row; the GPU must match it bit for
bit there (radii, pair lists, tile ranges, feature map, allmap, final T,
contributor counts), and the MLP decode within its tolerance.  For the 1M
scene the whole sorted pair list is compared; for the 4M scene (hundreds of
millions of pairs) the oracle's pairs are filtered to the sampled tile rows
and stable-sorted there, which is the same order the full stable sort gives
those tiles.  Whole-frame invariants cover the rows the oracle skips."""
import dataclasses

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _log(*a):
    print("[fullsize]", *a, flush=True)


def _gpu_frame(sc, cam_index):
    from nest_splat import rasterizer as rz
    from nest_splat.camera import view_ray_matrix
    from nest_splat.mlp import NestMLP
    sp = sc.spec
    cam = sc.cameras[cam_index]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets,
                           np.asarray(sp.gridrange, np.float32))
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), channels=sp.C)
    mlp = NestMLP(sp.C, sp.mlp_width, sp.mlp_dtype, sc.W1, sc.W2, sc.W3).to(DEV)
    bg = torch.tensor(sp.bg, dtype=torch.float32) if sum(sp.bg) > 0 else None
    rgb = mlp.decode_image(res.color, view_ray_matrix(cam), alpha=res.others[1], bg=bg)
    torch.cuda.synchronize()
    return res, rgb


def _sampled_rows(H, stride, phase):
    gy = (H + 15) // 16
    return [ty for ty in range(gy) if ty % stride == phase]


def _partial_binning(oracle, pre, W, H, rows):
    """Pairs of the tiles in `rows`, in the order the reference's stable sort
    gives them, with their ranges (other tiles empty)."""
    from oracle.oracle import lib as olib
    gx, gy = (W + 15) // 16, (H + 15) // 16
    P = pre["radii"].shape[0]
    offs = np.zeros(P, np.uint32)
    olib().or_inclusive_scan_u32(P, np.ascontiguousarray(pre["tiles"], np.uint32), offs)
    NR = int(offs[-1])
    keys = np.zeros(max(NR, 1), np.uint64)
    vals = np.zeros(max(NR, 1), np.uint32)
    olib().or_duplicate_keys(P, pre["xy"], pre["depth"], pre["radii"], offs, gx, gy, keys, vals)
    keys, vals = keys[:NR], vals[:NR]
    tile = (keys >> np.uint64(32)).astype(np.int64)
    sel = np.isin(tile // gx, rows)
    k, v = keys[sel], vals[sel]
    order = np.argsort(k, kind="stable")
    k, v = k[order], v[order]
    ranges = np.zeros((gx * gy, 2), np.uint32)
    t = (k >> np.uint64(32)).astype(np.int64)
    if t.size:
        starts = np.flatnonzero(np.r_[True, t[1:] != t[:-1]])
        ends = np.r_[starts[1:], t.size]
        ranges[t[starts], 0] = starts
        ranges[t[starts], 1] = ends
    return dict(num_rendered=NR, keys=k, vals=v, ranges=ranges)


def _check_rows(sc, cam_index, res, rgb, r, rows, oracle):
    sp = sc.spec
    cam = sc.cameras[cam_index]
    W, H = cam.image_width, cam.image_height
    pix = np.zeros((H, W), bool)
    for ty in rows:
        pix[ty * 16:(ty + 1) * 16] = True
    col = res.color.cpu().numpy()
    oth = res.others.cpu().numpy()
    from nest_splat import rasterizer as rz
    ba = rz.binning_arrays(res, W, H)
    ft = ba["final_T"].cpu().numpy()
    nc = ba["n_contrib"].cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(col[:, pix], r["color"][:, pix])
    np.testing.assert_array_equal(oth[:, pix], r["others"][:, pix])
    np.testing.assert_array_equal(ft[:, pix], r["final_T"][:, pix])
    np.testing.assert_array_equal(nc[:, pix], r["n_contrib"][:, pix])
    # MLP on the sampled pixels, tolerance of the bf16/fp16 MFMA path
    idx = np.flatnonzero(pix.reshape(-1))
    dirs = oracle.ray_dirs(cam)[idx]
    ref = oracle.mlp(np.ascontiguousarray(r["color"].reshape(sp.C, -1)[:, idx]), dirs,
                     r["others"][1].reshape(-1)[idx], sc.W1, sc.W2, sc.W3, sp.mlp_dtype,
                     np.asarray(sp.bg, np.float32), threads=0)
    got = rgb.cpu().numpy().reshape(3, -1)[:, idx]
    _log(f"MLP ({sp.mlp_dtype}) max abs error {np.abs(got - ref).max():.2e} over {idx.size} pixels")
    np.testing.assert_allclose(got, ref, atol=1e-3, rtol=0)
    # whole-frame invariants
    T = oth[1]
    assert np.all((T >= 0) & (T <= 1))
    np.testing.assert_array_equal(oth[1], 1 - ft[0])
    assert np.all(oth[7] >= 0) and np.all(oth[7] == np.floor(oth[7]))
    assert np.all(np.isfinite(col))
    return int(pix.sum())


def _full_binning_check(oracle, sc, res, pre, W, H):
    from nest_splat import rasterizer as rz
    b = oracle.binning(pre, W, H)
    np.testing.assert_array_equal(res.radii.cpu().numpy(), pre["radii"])
    assert res.num_rendered == b["num_rendered"]
    ba = rz.binning_arrays(res, W, H)
    np.testing.assert_array_equal(ba["keys"].cpu().numpy().view(np.uint64), b["keys"])
    np.testing.assert_array_equal(ba["vals"].cpu().numpy().view(np.uint32), b["vals"])
    np.testing.assert_array_equal(ba["ranges"].cpu().numpy().view(np.uint32), b["ranges"])
    return b


@pytest.mark.timeout(600)
def test_object_scene_100k(oracle):
    """The 100k-splat sphere shell at 800x800 with the 16-level 2^19 grid
    (dense levels 0-4, hashed 5-15), fp16 MLP, white background."""
    from nest_splat.scene import get_spec, make_scene
    sc = make_scene(get_spec("cfg2"))
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    _log("cfg2 GPU frame")
    res, rgb = _gpu_frame(sc, 0)
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = _full_binning_check(oracle, sc, res, pre, W, H)
    stride, phase = 4, 1
    _log("cfg2 oracle render, every", stride, "th tile row")
    grid = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, sp.C, grid, homotrans=sc.homotrans, ap_level=sc.ap_level, row_stride=stride,
                      row_phase=phase)
    n = _check_rows(sc, 0, res, rgb, r, _sampled_rows(H, stride, phase), oracle)
    hits = res.others[7].double().mean().item()
    _log(f"cfg2 ok, {n} pixels compared bit for bit, {res.num_rendered} pairs, {hits:.2f} hits/px")


@pytest.mark.timeout(600)
def test_rvq_scene_500k(oracle):
    """The 500k-splat scene whose scale, rotation and opacity are 4-stage RVQ
    codes into 4096-entry codebooks: decoded on the GPU (bit-exact with the
    oracle's ordered float32 sum and activations), then rendered at 800x800
    with the 2^19 grid and decoded by the fp16 MLP."""
    from nest_splat import rasterizer as rz
    from nest_splat.camera import view_ray_matrix
    from nest_splat.mlp import NestMLP
    from nest_splat.rvq import RVQAttributes
    from nest_splat.scene import RVQ_BIAS, build_homotrans_np, get_spec, make_scene
    sc = make_scene(get_spec("cfg4"))
    sp = sc.spec
    assert sp.rvq_codebook == 4096 and sp.P == 500_000
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    _log("cfg4 GPU decode")
    dec = RVQAttributes.from_numpy(sc.rvq_codebooks, sc.rvq_indices, RVQ_BIAS, DEV).decode()
    raw = {a: oracle.rvq_decode(sc.rvq_codebooks[a], sc.rvq_indices[a], RVQ_BIAS[a]) for a in RVQ_BIAS}
    scales, rots, op = oracle.activate(raw["scale"], raw["rotation"], raw["opacity"])
    np.testing.assert_array_equal(dec["scale"].cpu().numpy(), scales)
    np.testing.assert_array_equal(dec["rotation"].cpu().numpy(), rots)
    np.testing.assert_array_equal(dec["opacity"].cpu().numpy()[:, 0], op)
    homo = build_homotrans_np(rots, scales, sc.means)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32))
    _log("cfg4 GPU frame")
    res = rz.rasterize_forward(settings, grid, t(sc.means), dec["opacity"], dec["scale"], dec["rotation"],
                               homotrans=t(homo), ap_level=t(sc.ap_level), channels=sp.C)
    mlp = NestMLP(sp.C, sp.mlp_width, sp.mlp_dtype, sc.W1, sc.W2, sc.W3).to(DEV)
    rgb = mlp.decode_image(res.color, view_ray_matrix(cam), alpha=res.others[1],
                           bg=torch.tensor(sp.bg, dtype=torch.float32))
    torch.cuda.synchronize()
    pre = oracle.preprocess(sc.means, scales, rots, op[:, None], cam.world_view_transform, cam.full_proj_transform,
                            W, H)
    b = _full_binning_check(oracle, sc, res, pre, W, H)
    stride, phase = 5, 2
    _log("cfg4 oracle render, every", stride, "th tile row")
    g = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, sp.C, g, homotrans=homo, ap_level=sc.ap_level, row_stride=stride,
                      row_phase=phase)
    # the decoded scene's own arrays stand in for the generated ones in the row check
    sc2 = dataclasses.replace(sc, scales=scales, rotations=rots, opacity=op[:, None], homotrans=homo)
    n = _check_rows(sc2, 0, res, rgb, r, _sampled_rows(H, stride, phase), oracle)
    _log(f"cfg4 ok, {n} pixels compared bit for bit, {res.num_rendered} pairs")


@pytest.mark.timeout(600)
def test_benchmark_scene_1m(oracle):
    from nest_splat.scene import get_spec, make_scene
    from nest_splat import rasterizer as rz
    sc = make_scene(get_spec("cfg3"))
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    _log("cfg3 GPU frame")
    res, rgb = _gpu_frame(sc, 0)
    _log("cfg3 oracle preprocess + binning")
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    np.testing.assert_array_equal(res.radii.cpu().numpy(), pre["radii"])
    assert res.num_rendered == b["num_rendered"]
    ba = rz.binning_arrays(res, W, H)
    np.testing.assert_array_equal(ba["keys"].cpu().numpy().view(np.uint64), b["keys"])
    np.testing.assert_array_equal(ba["vals"].cpu().numpy().view(np.uint32), b["vals"])
    np.testing.assert_array_equal(ba["ranges"].cpu().numpy().view(np.uint32), b["ranges"])
    stride, phase = 8, 3
    _log("cfg3 oracle render, every", stride, "th tile row")
    grid = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, sp.C, grid, homotrans=sc.homotrans, ap_level=sc.ap_level, row_stride=stride,
                      row_phase=phase)
    n = _check_rows(sc, 0, res, rgb, r, _sampled_rows(H, stride, phase), oracle)
    _log("cfg3 ok,", n, "pixels compared bit for bit")


@pytest.mark.timeout(900)
@pytest.mark.parametrize("cam_index", range(8))
def test_stress_scene_4m(oracle, cam_index):
    from nest_splat.scene import get_spec, make_scene
    from nest_splat import rasterizer as rz
    global _cfg5
    try:
        sc = _cfg5
    except NameError:
        _log("cfg5 scene (4M splats)")
        sc = _cfg5 = make_scene(get_spec("cfg5"))
    sp = sc.spec
    cam = sc.cameras[cam_index]
    W, H = cam.image_width, cam.image_height
    _log(f"cfg5 cam {cam_index} GPU frame")
    res, rgb = _gpu_frame(sc, cam_index)
    _log(f"cfg5 cam {cam_index} oracle preprocess")
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    np.testing.assert_array_equal(res.radii.cpu().numpy(), pre["radii"])
    stride, phase = 16, (7 + 5 * cam_index) % 16
    rows = _sampled_rows(H, stride, phase)
    _log(f"cfg5 cam {cam_index} oracle pairs of tile rows {rows}")
    b = _partial_binning(oracle, pre, W, H, rows)
    assert res.num_rendered == b["num_rendered"]
    ba = rz.binning_arrays(res, W, H)
    granges = ba["ranges"].cpu().numpy().view(np.uint32)
    gvals = ba["vals"].cpu().numpy().view(np.uint32)
    gx = (W + 15) // 16
    for ty in rows:
        for tx in range(gx):
            ti = ty * gx + tx
            lo, hi = b["ranges"][ti]
            glo, ghi = granges[ti]
            assert ghi - glo == hi - lo, (ti, ghi - glo, hi - lo)
            np.testing.assert_array_equal(gvals[glo:ghi], b["vals"][lo:hi])
    # the whole sorted key array is ordered by (tile, depth bits)
    keys = ba["keys"].cpu().numpy().view(np.uint64)
    assert np.all(keys[1:] >= keys[:-1])
    _log(f"cfg5 cam {cam_index} oracle render of {len(rows)} tile rows")
    grid = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    r = oracle.render(pre, b, W, H, sp.C, grid, homotrans=sc.homotrans, ap_level=sc.ap_level, row_stride=stride,
                      row_phase=phase)
    n = _check_rows(sc, cam_index, res, rgb, r, rows, oracle)
    _log(f"cfg5 cam {cam_index} ok, {n} pixels compared bit for bit")


@pytest.mark.timeout(900)
@pytest.mark.parametrize("case", ["adaptive_cat_training", "general_kernel", "hybrid_sh"])
def test_benchmark_scene_1m_other_modes(oracle, case):
    """The 1M-splat frame in other configurations, bit for bit on every 16th
    tile row: render mode 12 in training with the first 10 levels as per-splat
    rows (weights in [0.15, 1)) and the last 6 as the grid, as bench.py
    --modes builds it; the general kernel (kernel_type 3, exponents 2-8); and
    render mode 8 over a one-level 3-channel grid at resolution 2048."""
    from nest_splat.scene import get_spec, make_scene
    from nest_splat import rasterizer as rz
    sc = make_scene(get_spec("cfg3"))
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy, cam.world_view_transform,
                                cam.full_proj_transform, cam.camera_center, if_contract=sp.contract)
    rng = np.random.default_rng(1)
    kw, okw = {}, {}
    if case == "adaptive_cat_training":
        hyb, F, Lt = 10, sp.F, sp.L
        offs = np.asarray(sc.offsets, np.int64)
        sub_offsets = offs[hyb:] - offs[hyb]
        sub_table = np.ascontiguousarray(sc.table[int(offs[hyb]):int(offs[Lt])])
        sub_base = int(round(2.0 ** (hyb * sp.S) * sp.base_res))
        rows = (rng.standard_normal((sp.P, Lt * F + 1)) * 0.1).astype(np.float32)
        rows[:, Lt * F] = rng.uniform(0.15, 1.0, sp.P).astype(np.float32)
        C = Lt * F
        grid = rz.HashGridDesc(Lt - hyb, F, sp.S, sub_base, t(sub_table), sub_offsets,
                               np.asarray(sp.gridrange, np.float32), render_mode=12, hybrid_levels=hyb,
                               total_levels=Lt)
        kw = dict(colors_precomp=t(rows))
        og = oracle.make_grid(Lt - hyb, F, sp.S, sub_base, sub_offsets, sub_table, sp.gridrange, sp.contract)
        okw = dict(colors=rows, render_mode=12, level=(Lt << 16) | ((Lt - hyb) << 8) | hyb)
    elif case == "general_kernel":
        C = sp.C
        shapes = rng.uniform(2.0, 8.0, sp.P).astype(np.float32)
        grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets,
                               np.asarray(sp.gridrange, np.float32))
        kw = dict(shapes=t(shapes), kernel_type=3)
        og = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
        okw = dict(shapes=shapes, kernel_type=3)
    else:
        C = 3
        table = rng.uniform(-0.5, 0.5, (1 << 21, 3)).astype(np.float32)
        hoffs = np.array([0, 1 << 21], np.int64)
        rows = rng.standard_normal((sp.P, 3)).astype(np.float32)
        grid = rz.HashGridDesc(1, 3, 0.0, 2048, t(table), hoffs, np.asarray(sp.gridrange, np.float32), render_mode=8)
        kw = dict(colors_precomp=t(rows))
        og = oracle.make_grid(1, 3, 0.0, 2048, hoffs, table, sp.gridrange, sp.contract)
        okw = dict(colors=rows, render_mode=8, level=(0 << 24) | (3 << 16) | (1 << 8))
    _log(f"cfg3 {case}: GPU frame")
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), channels=C, **kw)
    torch.cuda.synchronize()
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    assert res.num_rendered == b["num_rendered"]
    stride, phase = 16, 7
    _log(f"cfg3 {case}: oracle render, every {stride}th tile row")
    r = oracle.render(pre, b, W, H, C, og, homotrans=sc.homotrans, ap_level=sc.ap_level, row_stride=stride,
                      row_phase=phase, **okw)
    pix = np.zeros((H, W), bool)
    for ty in _sampled_rows(H, stride, phase):
        pix[ty * 16:(ty + 1) * 16] = True
    ba = rz.binning_arrays(res, W, H)
    np.testing.assert_array_equal(res.color.cpu().numpy()[:, pix], r["color"][:, pix])
    np.testing.assert_array_equal(res.others.cpu().numpy()[:, pix], r["others"][:, pix])
    np.testing.assert_array_equal(ba["n_contrib"].cpu().numpy().view(np.uint32)[:, pix], r["n_contrib"][:, pix])
    assert np.abs(r["color"][:, pix]).max() > 0
    _log(f"cfg3 {case} ok, {int(pix.sum())} pixels compared bit for bit")
