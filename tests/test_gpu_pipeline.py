"""GPU parity of the forward rasterizer against the CPU oracle, stage by stage.

Integer results (radii, tiles touched, pair offsets, sort keys and values,
tile ranges, per-pixel hit counts, contributor counts) must be bit-exact.
Float maps share the oracle's evaluation order, so they are compared bit for
bit as well, and additionally against the stated tolerance (feature map 1e-5
relative to the map's magnitude).
"""
import numpy as np
import pytest
import torch

from scenes import scene

pytestmark = pytest.mark.gpu

SCENES = ["cfg1", "shell_small", "unbounded_small", "shells_small"]


def run_gpu(sc, cam_index=0, max_intersections=0, align_corners=False, interp=0, beta=0.0, record=False,
            kernel_type=0, shapes=None):
    from nest_splat import rasterizer as rz
    sp = sc.spec
    cam = sc.cameras[cam_index]
    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    settings = rz.make_settings(cam.image_height, cam.image_width, cam.tanfovx, cam.tanfovy,
                                cam.world_view_transform, cam.full_proj_transform, cam.camera_center,
                                beta=beta, if_contract=sp.contract, max_intersections=max_intersections)
    grid = rz.HashGridDesc(sp.L, sp.F, sp.S, sp.base_res, t(sc.table), sc.offsets, np.asarray(sp.gridrange, np.float32),
                           align_corners=align_corners, interpolation=interp)
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               homotrans=t(sc.homotrans), ap_level=t(sc.ap_level), channels=sp.C,
                               record_transmittance=record, kernel_type=kernel_type,
                               shapes=None if shapes is None else t(shapes))
    torch.cuda.synchronize()
    return res


def run_oracle(O, sc, cam_index=0, max_intersections=0, align_corners=False, interp=0, beta=0.0, record=False,
               kernel_type=0, shapes=None):
    sp = sc.spec
    cam = sc.cameras[cam_index]
    W, H = cam.image_width, cam.image_height
    pre = O.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                       cam.full_proj_transform, W, H)
    b = O.binning(pre, W, H)
    grid = O.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract,
                       align_corners=align_corners, interp=interp)
    r = O.render(pre, b, W, H, sp.C, grid, homotrans=sc.homotrans, ap_level=sc.ap_level,
                 max_intersections=max_intersections, beta=beta, record_transmittance=record,
                 kernel_type=kernel_type, shapes=shapes)
    return pre, b, r


def depth_ordered_pairs(pre, b):
    """Splat order by (depth bits, index) with culled splats last, tiles
    touched in that order, and for each depth-ordered pair its position in
    the oracle's splat-ordered pair list."""
    vis = pre["radii"] > 0
    dkey = np.where(vis, pre["depth"].astype(np.float32).view(np.uint32), np.uint32(0xFFFFFFFF))
    order = np.argsort(dkey, kind="stable").astype(np.uint32)
    tiles = pre["tiles"].astype(np.int64)
    starts = b["offsets"].astype(np.int64) - tiles  # inclusive scan -> first pair of each splat
    lens = tiles[order]
    NR = int(lens.sum())
    src = np.repeat(starts[order] - (np.cumsum(lens) - lens), lens) + np.arange(NR)
    return order, lens.astype(np.uint32), src


@pytest.mark.parametrize("name", SCENES)
def test_preprocess_binning_render_parity(oracle, name):
    from nest_splat import rasterizer as rz
    sc = scene(name)
    print(f"[case] {name} P={sc.spec.P} {sc.spec.W}x{sc.spec.H}", flush=True)
    res = run_gpu(sc)
    pre, b, r = run_oracle(oracle, sc)
    P = sc.spec.P
    ga = {k: v.cpu().numpy() for k, v in rz.geometry_arrays(res, P).items()}
    radii = res.radii.cpu().numpy()
    np.testing.assert_array_equal(radii, pre["radii"])
    np.testing.assert_array_equal(ga["radii"], pre["radii"])
    np.testing.assert_array_equal(ga["tiles"].view(np.uint32), pre["tiles"])
    vis = pre["radii"] > 0
    assert vis.sum() > 0
    np.testing.assert_array_equal(ga["xy"][vis], pre["xy"][vis])
    np.testing.assert_array_equal(ga["depth"][vis], pre["depth"][vis])
    rec = ga["records"][vis]
    np.testing.assert_array_equal(rec[:, 0:9], pre["transmat"][vis])
    np.testing.assert_array_equal(rec[:, 11], pre["normal_opacity"][vis][:, 3])
    np.testing.assert_array_equal(rec[:, 12:15], pre["normal_opacity"][vis][:, :3])
    np.testing.assert_array_equal(ga["offsets"].view(np.uint32), b["offsets"])

    assert res.num_rendered == b["num_rendered"]
    ba = {k: v.cpu().numpy() for k, v in rz.binning_arrays(res, sc.spec.W, sc.spec.H).items()}
    # intermediate of the depth-first binning: the oracle's splat-ordered
    # pairs regrouped splat by splat in (depth bits, index) order
    order, lens, src = depth_ordered_pairs(pre, b)
    np.testing.assert_array_equal(ga["depth_order"].view(np.uint32), order)
    np.testing.assert_array_equal(ga["order_offsets"].view(np.uint32), np.cumsum(lens) - lens)
    np.testing.assert_array_equal(ba["pair_tiles"].view(np.uint32), (b["keys_unsorted"][src] >> 32).astype(np.uint32))
    np.testing.assert_array_equal(ba["pair_ids"].view(np.uint32), b["vals_unsorted"][src])
    np.testing.assert_array_equal(ba["keys"].view(np.uint64), b["keys"])
    np.testing.assert_array_equal(ba["vals"].view(np.uint32), b["vals"])
    np.testing.assert_array_equal(ba["ranges"].view(np.uint32), b["ranges"])

    others = res.others.cpu().numpy()
    color = res.color.cpu().numpy()
    np.testing.assert_array_equal(others[7], r["others"][7])  # hit counts
    np.testing.assert_array_equal(ba["n_contrib"].view(np.uint32), r["n_contrib"])
    np.testing.assert_array_equal(ba["final_T"], r["final_T"])
    np.testing.assert_array_equal(others, r["others"])
    scale = max(np.abs(r["color"]).max(), 1e-30)
    np.testing.assert_allclose(color, r["color"], rtol=1e-5, atol=1e-5 * scale)
    np.testing.assert_array_equal(color, r["color"])


def test_max_intersections_parity(oracle):
    sc = scene("shell_small")
    res = run_gpu(sc, max_intersections=3)
    _, _, r = run_oracle(oracle, sc, max_intersections=3)
    hits = res.others.cpu().numpy()[7]
    np.testing.assert_array_equal(hits, r["others"][7])
    assert hits.max() <= 3
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


def test_second_camera_parity(oracle):
    sc = scene("shells_small")
    res = run_gpu(sc, cam_index=1)
    _, b, r = run_oracle(oracle, sc, cam_index=1)
    assert res.num_rendered == b["num_rendered"]
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


@pytest.mark.parametrize("sizes,name", [("non_pow2", "unbounded_small"), ("mixed", "shells_small")])
def test_irregular_level_sizes_parity(oracle, sizes, name):
    """Level sizes that are not all powers of two (hashed levels reduced by a
    modulo, a hashed level between dense ones): the render takes the general
    per-level index path instead of the dense-prefix/power-of-two one."""
    import dataclasses
    sc = scene(name)  # f32 and f16 tables
    L, T = sc.spec.L, 1 << sc.spec.log2T
    if sizes == "non_pow2":
        hs = np.full(L, T - 40, np.int64)
    else:  # power-of-two and other sizes alternating; level 1 hashed into 64 entries
        hs = np.where(np.arange(L) % 2 == 0, T, T - 8 * 37).astype(np.int64)
        hs[1] = 64
    offsets = np.concatenate([[0], np.cumsum(hs)]).astype(np.int32)
    rng = np.random.default_rng(7)
    table = (rng.standard_normal((int(offsets[-1]), sc.spec.F)) * 0.5).astype(sc.table.dtype)
    sc2 = dataclasses.replace(sc, offsets=offsets, table=table)
    print(f"[case] irregular level sizes {sizes} {name} {table.dtype} P={sc.spec.P}", flush=True)
    res = run_gpu(sc2)
    _, b, r = run_oracle(oracle, sc2)
    assert res.num_rendered == b["num_rendered"]
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


@pytest.mark.parametrize("name,align,interp", [("unbounded_small", False, 1), ("shell_small", True, 0),
                                               ("shells_small", True, 1), ("unbounded_small", True, 0)])
def test_align_corners_and_smoothstep_parity(oracle, name, align, interp):
    """align_corners (pos offset 0, resolution cells) and smoothstep
    weights (hashgrid.h smoothstep) take the general per-level path (its cell
    fraction is x - floor(x), also for a contracted coordinate that rounds
    below 0); trilinear grids without align_corners the dense-prefix/
    power-of-two one.  The contracted scene with align_corners and far splats
    is the case where the two would differ if a coordinate fell below 0."""
    sc = scene(name)
    print(f"[case] {name} align_corners={align} interp={interp}", flush=True)
    res = run_gpu(sc, align_corners=align, interp=interp)
    _, b, r = run_oracle(oracle, sc, align_corners=align, interp=interp)
    assert res.num_rendered == b["num_rendered"]
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


@pytest.mark.parametrize("name,beta", [("shell_small", 0.5), ("unbounded_small", 4.0)])
def test_beta_activation_parity(oracle, name, beta):
    """G -> (1+beta) G / (1+beta G) (CR/forward.cu:915-916): hits with alpha in
    [1/255, ...) beyond the beta = 0 cut must be kept, so the render's early
    reject uses the beta-aware bound."""
    sc = scene(name)
    print(f"[case] {name} beta={beta}", flush=True)
    res = run_gpu(sc, beta=beta)
    _, b, r = run_oracle(oracle, sc, beta=beta)
    _, _, r0 = run_oracle(oracle, sc)
    assert (r["others"][7] > r0["others"][7]).any()  # beta accepts more hits than beta = 0
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])


def test_deterministic_repeat():
    sc = scene("unbounded_small")
    a = run_gpu(sc)
    b = run_gpu(sc)
    assert torch.equal(a.color, b.color) and torch.equal(a.others, b.others)


@pytest.mark.parametrize("name", ["cfg1", "unbounded_small", "shells_small"])
def test_tile_launch_order(name):
    """The render's launch order is a permutation of the tiles, heaviest
    first: in the order's positions the buckets of 8 log2(pairs + 1) do not
    increase (float32 log2 on the device may put a boundary weight one bucket
    off).  Workgroup b runs on XCD b % 8, and within each group of 8 * 16
    positions XCD x takes the run of 16 positions from 16 x on, so position pos
    is workgroup ((pos // 128) * 16 + pos % 16) * 8 + (pos % 128) // 16 (the
    tail after the last full group keeps pos)."""
    from nest_splat import rasterizer as rz
    sc = scene(name)
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    res = run_gpu(sc)
    ba = rz.binning_arrays(res, W, H)
    by_wg = ba["tile_order"].cpu().numpy().astype(np.int64)
    ranges = ba["ranges"].cpu().numpy().view(np.uint32).astype(np.int64)
    ntiles = ranges.shape[0]
    np.testing.assert_array_equal(np.sort(by_wg), np.arange(ntiles))
    pos = np.arange(ntiles)
    full = ntiles // 128 * 128
    wg = np.where(pos < full, ((pos // 128) * 16 + pos % 16) * 8 + (pos % 128) // 16, pos)
    np.testing.assert_array_equal(np.sort(wg), pos)  # a permutation
    order = by_wg[wg]
    w = ranges[:, 1] - ranges[:, 0]
    bucket = np.minimum(255, np.floor(8.0 * np.log2(w.astype(np.float64) + 1.0))).astype(np.int64)
    b = bucket[order]
    assert np.all(np.diff(b) <= 1) and b[0] >= bucket.max() - 1
    assert np.all(np.maximum.accumulate(b[::-1])[::-1] <= b + 1)


def check_record(res, r):
    """record_transmittance: hit counts exact, transmittance sums within 1e-5
    of the largest (the GPU sums per wave, the oracle per pixel)."""
    cover = res.cover_pixels.cpu().numpy()
    trans = res.trans_avg.cpu().numpy()
    np.testing.assert_array_equal(cover, r["cover_pixels"])
    scale = max(float(np.abs(r["trans_avg"]).max()), 1e-30)
    np.testing.assert_allclose(trans, r["trans_avg"], rtol=1e-5, atol=1e-6 * scale)
    assert cover.sum() > 0


@pytest.mark.parametrize("name,mx", [("cfg1", 0), ("shell_small", 0), ("unbounded_small", 0), ("shell_small", 5)])
def test_record_transmittance_parity(oracle, name, mx):
    """record_transmittance=True (CR/forward.cu:1961-1964): per-splat hit
    counts bit-exact, transmittance sums within tolerance, and the frame's
    other outputs unchanged by the recording."""
    sc = scene(name)
    print(f"[case] record_transmittance {name} max_intersections={mx}", flush=True)
    res = run_gpu(sc, max_intersections=mx, record=True)
    pre, b, r = run_oracle(oracle, sc, max_intersections=mx, record=True)
    check_record(res, r)
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    plain = run_gpu(sc, max_intersections=mx)
    assert plain.cover_pixels is None and plain.trans_avg is None
    np.testing.assert_array_equal(plain.color.cpu().numpy(), res.color.cpu().numpy())
    np.testing.assert_array_equal(plain.others.cpu().numpy(), res.others.cpu().numpy())
    # splats culled or off-screen record nothing
    assert not res.cover_pixels.cpu().numpy()[pre["radii"] == 0].any()


def test_record_transmittance_colour_path(oracle):
    """The colour path (no grid) records the same way."""
    from nest_splat import rasterizer as rz
    sc = scene("shell_small")
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    print("[case] record_transmittance colour path", flush=True)
    cols = np.random.default_rng(1).uniform(0, 1, (sp.P, 3)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))
    settings = rz.make_settings(H, W, cam.tanfovx, cam.tanfovy, cam.world_view_transform, cam.full_proj_transform,
                                cam.camera_center, if_contract=sp.contract)
    grid = rz.HashGridDesc(0, 1, 0.0, 0, None, np.zeros(1, np.int64), np.zeros(2, np.float32))
    res = rz.rasterize_forward(settings, grid, t(sc.means), t(sc.opacity), t(sc.scales), t(sc.rotations),
                               colors_precomp=t(cols), channels=3, record_transmittance=True)
    torch.cuda.synchronize()
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    r = oracle.render(pre, b, W, H, 3, None, colors=cols, record_transmittance=True)
    check_record(res, r)


def _shapes(kt, P, seed):
    """Per-splat kernel parameters in the ranges the reference trains them in:
    beta-kernel shapes around 1-4, flex betas 0-2 (some exactly 0), general
    exponents 2-8 (plus a few below 2)."""
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


@pytest.mark.parametrize("name,kt", [("cfg1", 1), ("shell_small", 2), ("unbounded_small", 3), ("shell_small", 1),
                                     ("cfg1", 3)])
def test_kernel_types_parity(oracle, name, kt):
    """kernel_type 1 (beta), 2 (flex) and 3 (general) (CR/forward.cu:864-900):
    the frame bit-exact against the oracle, the preprocess bounds of the
    render's early rejects conservative (no hit missed), and the
    transmittance record with them."""
    sc = scene(name)
    shapes = _shapes(kt, sc.spec.P, kt * 31 + len(name))
    print(f"[case] kernel_type {kt} {name}", flush=True)
    res = run_gpu(sc, kernel_type=kt, shapes=shapes, record=True)
    pre, b, r = run_oracle(oracle, sc, kernel_type=kt, shapes=shapes, record=True)
    from nest_splat import rasterizer as rz
    W, H = r["color"].shape[2], r["color"].shape[1]
    ba = {k: v.cpu().numpy() for k, v in rz.binning_arrays(res, W, H).items()}
    np.testing.assert_array_equal(res.others.cpu().numpy(), r["others"])
    np.testing.assert_array_equal(ba["n_contrib"].view(np.uint32), r["n_contrib"])
    np.testing.assert_array_equal(ba["final_T"], r["final_T"])
    np.testing.assert_array_equal(res.color.cpu().numpy(), r["color"])
    check_record(res, r)
    gauss = run_gpu(sc)
    assert not np.array_equal(gauss.others.cpu().numpy()[7], r["others"][7])  # the kernel changed the hits
