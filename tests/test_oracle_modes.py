"""Pins the oracle's render modes 4 (cat) and 13 (adaptive_cat_fast) on the
mode-0 oracle, which the golden vectors and the autograd tests pin.

Both modes compose each hit's feature vector from a per-splat feature row
and the grid (CR/forward.cu:965-1101, :1218-1282) and then blend it like
mode 0.  So every channel of their output is, per hit, either a row entry
(what the colour path blends), a grid feature (what mode 0 blends) or an
affine mix of the two, and the auxiliary outputs are mode 0's with the
mode's own omissions.  The tests render the same scene in the colour path
and in mode 0 with selected rows and levels masked out (a row of zeros
contributes nothing; ap_level 0 queries no level) and check:
  - bit-exact equality where a channel takes one source for every hit;
  - for hits that mix sources or splats that take different sources, the
    sum of the masked renders (float32 sums in a different order: 1e-5 of
    the map's largest entry);
  - the mode-specific outputs: mode 13 writes no appearance colour and no
    last contributor, and its weight > 0.5 inference hits add no world
    position.
"""
import numpy as np
import pytest

from nest_splat.scene import get_spec, make_scene

TOL = 1e-5


def _tiny(L=4, F=4, P=400, W=64, H=48, seed=0):
    spec = get_spec("cfg1", P=P, W=W, H=H, L=L, F=F, log2T=12, log_scale_mu=-2.2, name=f"modes{seed}_{L}_{F}")
    return make_scene(spec)


class _Frame:
    def __init__(self, oracle, sc):
        self.O, self.sc = oracle, sc
        sp = sc.spec
        cam = sc.cameras[0]
        self.W, self.H = cam.image_width, cam.image_height
        self.pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                                     cam.full_proj_transform, self.W, self.H)
        self.b = oracle.binning(self.pre, self.W, self.H)
        assert self.b["num_rendered"] > 0
        self.L, self.F, self.P = sp.L, sp.F, sp.P

    def grid(self, L=None):
        sp = self.sc.spec
        return self.O.make_grid(self.L if L is None else L, sp.F, sp.S, sp.base_res, self.sc.offsets, self.sc.table,
                                sp.gridrange, sp.contract)

    def colour(self, rows):
        rows = np.ascontiguousarray(rows, np.float32)
        return self.O.render(self.pre, self.b, self.W, self.H, rows.shape[1], None, colors=rows)

    def mode0(self, L=None, ap=None):
        L = self.L if L is None else L
        ap = self.sc.ap_level if ap is None else ap
        return self.O.render(self.pre, self.b, self.W, self.H, L * self.F, self.grid(L), homotrans=self.sc.homotrans,
                             ap_level=ap)

    def mode(self, render_mode, level, C, rows, L=None):
        return self.O.render(self.pre, self.b, self.W, self.H, C, self.grid(L), homotrans=self.sc.homotrans,
                             ap_level=self.sc.ap_level, colors=np.ascontiguousarray(rows, np.float32),
                             render_mode=render_mode, level=level)


def _same(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _close(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(np.abs(b).max(), 1e-30)
    return float(np.abs(a - b).max() / scale) <= TOL


@pytest.fixture(scope="module")
def frame(oracle):
    return _Frame(oracle, _tiny())


def test_mode4_without_splat_levels_is_mode0(frame):
    fr = frame
    L, F = fr.L, fr.F
    r4 = fr.mode(4, (L << 16) | (L << 8), L * F, np.zeros((fr.P, 0), np.float32))
    r0 = fr.mode0()
    for k in ("color", "others", "final_T", "n_contrib"):
        assert _same(r4[k], r0[k]) if k != "n_contrib" else np.array_equal(r4[k], r0[k]), k


@pytest.mark.parametrize("hyb", [1, 3])
def test_mode4_is_rows_then_grid(frame, hyb):
    fr = frame
    L, F = fr.L, fr.F
    pgd = hyb * F
    rows = np.random.default_rng(hyb).uniform(-1, 1, (fr.P, pgd)).astype(np.float32)
    C = pgd + L * F + 3  # three channels past the features stay zero
    r4 = fr.mode(4, ((hyb + L) << 16) | (1 << 8) | hyb, C, rows)
    rc = fr.colour(rows)
    r0 = fr.mode0()
    assert np.abs(r4["color"][:pgd]).max() > 0 and np.abs(r4["color"][pgd:pgd + L * F]).max() > 0
    assert _same(r4["color"][:pgd], rc["color"])
    assert _same(r4["color"][pgd:pgd + L * F], r0["color"])
    assert not np.any(r4["color"][pgd + L * F:])
    assert _same(r4["others"], r0["others"])
    assert _same(r4["final_T"], r0["final_T"])
    assert np.array_equal(r4["n_contrib"], r0["n_contrib"])


def test_mode4_grid_levels_from_offsets(oracle):
    """Mode 4 counts the grid's levels from the offsets (the last increasing
    entry), not from bits 8-15 of level: a grid whose last level is empty
    renders like its first L-1 levels."""
    sc = _tiny(L=3, F=2, seed=1)
    fr = _Frame(oracle, sc)
    offs = np.asarray(sc.offsets, np.int64).copy()
    offs[3] = offs[2]  # level 2 has no entries
    sp = sc.spec
    g = oracle.make_grid(3, sp.F, sp.S, sp.base_res, offs, sc.table, sp.gridrange, sp.contract)
    rows = np.random.default_rng(3).uniform(-1, 1, (fr.P, 2)).astype(np.float32)
    r4 = oracle.render(fr.pre, fr.b, fr.W, fr.H, 8, g, homotrans=sc.homotrans, ap_level=sc.ap_level, colors=rows,
                       render_mode=4, level=(4 << 16) | (3 << 8) | 1)
    r0 = fr.mode0(L=2)
    assert _same(r4["color"][2:6], r0["color"])
    assert not np.any(r4["color"][6:])


def test_drop_in_counts_cat_levels_like_the_oracle():
    import diff_surfel_rasterization as dsr
    offs = np.zeros(17, np.int64)
    offs[:5] = [0, 10, 30, 30, 70]
    assert dsr._cat_hash_levels(offs) == 4
    offs[:5] = [0, 10, 30, 70, 70]
    assert dsr._cat_hash_levels(offs) == 3
    assert dsr._cat_hash_levels(np.zeros(17, np.int64)) == 0


def _rows13(fr, hyb, extra, weights):
    total = hyb + fr.L + extra
    tdim = total * fr.F
    rows = np.random.default_rng(7).uniform(-1, 1, (fr.P, tdim + 1)).astype(np.float32)
    rows[:, tdim] = weights
    return rows, total, tdim


def test_mode13_inference_fast_takes_the_rows(frame):
    fr = frame
    hyb = 2
    rows, total, tdim = _rows13(fr, hyb, 1, 0.9)
    r = fr.mode(13 | 0x100, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    rc = fr.colour(rows[:, :tdim])
    assert _same(r["color"], rc["color"])
    assert _same(r["others"][:8], rc["others"][:8])
    assert not np.any(r["others"][8:])  # no world position, no appearance colour
    assert _same(r["final_T"], rc["final_T"])
    assert not np.any(r["n_contrib"][0])  # mode 13 never records the last contributor
    assert np.array_equal(r["n_contrib"][1], rc["n_contrib"][1])


def test_mode13_inference_slow_is_rows_then_grid(frame):
    fr = frame
    hyb = 2
    rows, total, tdim = _rows13(fr, hyb, 1, 0.3)
    pgd = hyb * fr.F
    r = fr.mode(13 | 0x100, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    rc = fr.colour(rows[:, :pgd])
    r0 = fr.mode0()
    assert _same(r["color"][:pgd], rc["color"])
    assert _same(r["color"][pgd:pgd + fr.L * fr.F], r0["color"])
    assert not np.any(r["color"][pgd + fr.L * fr.F:])  # row levels past the grid's are not taken
    assert _same(r["others"][:11], r0["others"][:11])
    assert not np.any(r["others"][11:])
    assert _same(r["final_T"], r0["final_T"])
    assert not np.any(r["n_contrib"][0])


def test_mode13_inference_mixed_weights(frame):
    fr = frame
    hyb = 1
    wts = np.random.default_rng(9).uniform(0, 1, fr.P).astype(np.float32)
    rows, total, tdim = _rows13(fr, hyb, 0, wts)
    pgd = hyb * fr.F
    fast = wts > 0.5
    assert 0.2 < fast.mean() < 0.8
    r = fr.mode(13 | 0x100, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    assert _same(r["color"][:pgd], fr.colour(rows[:, :pgd])["color"])
    fine_rows = np.where(fast[:, None], rows[:, pgd:tdim], 0.0)
    ap = np.where(fast, 0.0, fr.sc.ap_level.reshape(-1)).astype(np.float32)
    expect = fr.colour(fine_rows)["color"].astype(np.float64) + fr.mode0(ap=ap)["color"]
    assert _close(r["color"][pgd:], expect)


@pytest.mark.parametrize("t", [1.0, 0.0])
def test_mode13_training_weight_extremes(frame, t):
    fr = frame
    hyb = 2
    rows, total, tdim = _rows13(fr, hyb, 1, t)
    pgd, nf = hyb * fr.F, fr.L * fr.F
    r = fr.mode(13, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    r0 = fr.mode0()
    if t == 1.0:
        assert _same(r["color"][:pgd + nf], fr.colour(rows[:, :pgd + nf])["color"])
    else:
        assert not np.any(r["color"][:pgd])
        assert _same(r["color"][pgd:pgd + nf], r0["color"])
    assert not np.any(r["color"][pgd + nf:])
    assert _same(r["others"][:11], r0["others"][:11])
    assert not np.any(r["others"][11:])
    assert not np.any(r["n_contrib"][0])


def test_mode13_training_per_splat_weights(frame):
    """Three groups of splats with weights 0.2, 0.55, 0.9: each group's
    share is t * (its rows) + (1 - t) * (its grid features)."""
    fr = frame
    hyb = 2
    ts = np.array([0.2, 0.55, 0.9], np.float32)
    grp = np.arange(fr.P) % 3
    rows, total, tdim = _rows13(fr, hyb, 0, ts[grp])
    pgd, nf = hyb * fr.F, fr.L * fr.F
    r = fr.mode(13, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    expect = np.zeros((tdim,) + r["color"].shape[1:], np.float64)
    for k, t in enumerate(ts):
        mine = grp == k
        ap = np.where(mine, fr.sc.ap_level.reshape(-1), 0.0).astype(np.float32)
        part = fr.colour(np.where(mine[:, None], rows[:, :tdim] * t, 0.0))["color"].astype(np.float64)
        part[pgd:] += (1.0 - float(t)) * fr.mode0(ap=ap)["color"]
        expect += part
    assert _close(r["color"], expect)


@pytest.mark.parametrize("t", [1.0, 0.0])
def test_mode12_training_weight_extremes(frame, t):
    """adaptive_cat training (CR/forward.cu:1676-1711): the row's first hyb*F
    channels unweighted, the next grid levels blended; every hit is a full
    one, so the auxiliary outputs are mode 0's."""
    fr = frame
    hyb = 2
    rows, total, tdim = _rows13(fr, hyb, 1, t)
    pgd, nf = hyb * fr.F, fr.L * fr.F
    r = fr.mode(12, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    r0 = fr.mode0()
    if t == 1.0:
        assert _same(r["color"][:pgd + nf], fr.colour(rows[:, :pgd + nf])["color"])
    else:
        assert _same(r["color"][:pgd], fr.colour(rows[:, :pgd])["color"])
        assert _same(r["color"][pgd:pgd + nf], r0["color"])
    assert not np.any(r["color"][pgd + nf:])
    assert _same(r["others"], r0["others"])
    assert _same(r["final_T"], r0["final_T"])
    assert np.array_equal(r["n_contrib"], r0["n_contrib"])
    assert r["n_contrib"][0].any()


def test_mode12_training_per_splat_weights(frame):
    fr = frame
    hyb = 1
    ts = np.array([0.25, 0.6, 0.85], np.float32)
    grp = np.arange(fr.P) % 3
    rows, total, tdim = _rows13(fr, hyb, 0, ts[grp])
    pgd = hyb * fr.F
    r = fr.mode(12, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
    assert _same(r["color"][:pgd], fr.colour(rows[:, :pgd])["color"])
    expect = np.zeros((tdim - pgd,) + r["color"].shape[1:], np.float64)
    for k, t in enumerate(ts):
        mine = grp == k
        ap = np.where(mine, fr.sc.ap_level.reshape(-1), 0.0).astype(np.float32)
        expect += fr.colour(np.where(mine[:, None], rows[:, pgd:tdim] * t, 0.0))["color"]
        expect += (1.0 - float(t)) * fr.mode0(ap=ap)["color"]
    assert _close(r["color"][pgd:], expect)


def test_mode12_inference_threshold(frame):
    """adaptive_cat inference (CR/forward.cu:1636-1675): weight >= 0.9 takes
    the whole row (0.9 itself included), below takes the grid; unlike mode
    13 the hits keep their world position, appearance colour and last
    contributor."""
    fr = frame
    hyb = 2
    pgd, nf = hyb * fr.F, fr.L * fr.F
    r0 = fr.mode0()
    for wt, fast in ((0.9, True), (0.97, True), (np.nextafter(np.float32(0.9), np.float32(0)), False)):
        rows, total, tdim = _rows13(fr, hyb, 1, wt)
        r = fr.mode(12 | 0x100, (total << 16) | (fr.L << 8) | hyb, tdim, rows)
        if fast:
            assert _same(r["color"], fr.colour(rows[:, :tdim])["color"])
        else:
            assert _same(r["color"][:pgd], fr.colour(rows[:, :pgd])["color"])
            assert _same(r["color"][pgd:pgd + nf], r0["color"])
            assert not np.any(r["color"][pgd + nf:])
        assert _same(r["others"], r0["others"])
        assert np.array_equal(r["n_contrib"], r0["n_contrib"])


def test_mode14_adaptive_zero(frame):
    """adaptive_zero (CR/forward.cu:1716-1830): rows [hyb*F | weight]; the
    grid levels times the weight when it is > 1e-6 (training) or >= 0.1
    (inference), else zero; full hits (auxiliary outputs of mode 0)."""
    fr = frame
    hyb, L, F = 2, fr.L, fr.F
    pgd, nf = hyb * F, L * F
    total = hyb + L + 1
    tdim = total * F
    level = (total << 16) | (L << 8) | hyb
    r0 = fr.mode0()
    base = np.random.default_rng(11).uniform(-1, 1, (fr.P, pgd + 1)).astype(np.float32)
    for mode, wt, on in ((14, 1.0, True), (14, 1e-6, False), (14 | 0x100, 0.1, True),
                         (14 | 0x100, np.nextafter(np.float32(0.1), np.float32(0)), False)):
        rows = base.copy()
        rows[:, pgd] = wt
        r = fr.mode(mode, level, tdim, rows)
        assert _same(r["color"][:pgd], fr.colour(rows[:, :pgd])["color"])
        if on and wt == 1.0:
            assert _same(r["color"][pgd:pgd + nf], r0["color"])
        elif on:
            assert _close(r["color"][pgd:pgd + nf], np.float32(wt) * r0["color"].astype(np.float64))
        else:
            assert not np.any(r["color"][pgd:])
        assert not np.any(r["color"][pgd + nf:])
        assert _same(r["others"], r0["others"])
        assert np.array_equal(r["n_contrib"], r0["n_contrib"])


@pytest.mark.parametrize("t", [1.0, 0.0])
def test_mode7_adaptive_add_weight_extremes(frame, t):
    """adaptive_add (CR/forward.cu:1326-1376): every channel is
    weight * row + (1 - weight) * grid, the grid zero past its levels; full
    hits."""
    fr = frame
    rows, total, tdim = _rows13(fr, 0, 2, t)
    nf = fr.L * fr.F
    r = fr.mode(7, (total << 16) | (fr.L << 8), tdim, rows)
    r0 = fr.mode0()
    if t == 1.0:
        assert _same(r["color"], fr.colour(rows[:, :tdim])["color"])
    else:
        assert _same(r["color"][:nf], r0["color"])
        assert not np.any(r["color"][nf:])
    assert _same(r["others"], r0["others"])
    assert np.array_equal(r["n_contrib"], r0["n_contrib"])
