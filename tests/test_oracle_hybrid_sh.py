"""Pins the oracle's hybrid SH render modes 8 (hybrid_SH), 9 (hybrid_SH_post)
and 10 (hybrid_SH_raw) (CR/forward.cu:1378-1542) on its colour path and its
mode-0 grid path, which the golden vectors and the autograd tests pin.

Each hit's channels come from the splat's row (3 raw SH colours, or 48 SH
coefficients) and one 3-channel grid level at the hit, combined per hit:
  - with decompose 1 (gaussian_only) the grid is left out, so the colours are
    the colour path's over the activated rows (bit-exact);
  - mode 9 is linear: the non-DC channels are the colour path's (bit-exact),
    the DC channels the colour path's plus mode 0's grid (float32 sums in
    another order: 1e-5 of the map's largest entry), or mode 0's grid alone
    with decompose 2 (bit-exact);
  - modes 8 and 10 activate per hit, so pixels with a single hit are checked
    against the closed form: their mode-0 grid value is h * alpha, their
    output f(raw, h) * alpha (relative 1e-5: alpha comes back from 1 - T and
    h from a division);
  - every mode records the world position and appearance colour as mode 0's
    grid path does.
"""
import numpy as np
import pytest

from nest_splat.scene import get_spec, make_scene

f32 = np.float32
TOL = 1e-5


class _Frame:
    def __init__(self, oracle, base_res):
        spec = get_spec("cfg1", P=300, W=64, H=48, L=1, F=3, log2T=12, base_res=base_res, log_scale_mu=-2.2,
                        name=f"hsh{base_res}")
        sc = self.sc = make_scene(spec)
        self.O = oracle
        cam = sc.cameras[0]
        self.W, self.H = cam.image_width, cam.image_height
        self.pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                                     cam.full_proj_transform, self.W, self.H)
        self.b = oracle.binning(self.pre, self.W, self.H)
        assert self.b["num_rendered"] > 0
        rng = np.random.default_rng(base_res)
        self.raw = rng.normal(0.0, 1.2, (spec.P, 3)).astype(f32)
        self.sh = rng.normal(0.0, 0.5, (spec.P, 48)).astype(f32)
        self.grid = oracle.make_grid(1, 3, spec.S, spec.base_res, sc.offsets, sc.table, spec.gridrange, spec.contract)

    def colour(self, rows):
        rows = np.ascontiguousarray(rows, f32)
        return self.O.render(self.pre, self.b, self.W, self.H, rows.shape[1], None, colors=rows)

    def mode0(self):
        return self.O.render(self.pre, self.b, self.W, self.H, 3, self.grid, homotrans=self.sc.homotrans,
                             ap_level=self.sc.ap_level)

    def hsh(self, mode, dec, hl=1):
        rows = self.sh if mode == 9 else self.raw
        return self.O.render(self.pre, self.b, self.W, self.H, 48 if mode == 9 else 3, self.grid,
                             homotrans=self.sc.homotrans, ap_level=self.sc.ap_level, colors=rows, render_mode=mode,
                             level=(dec << 24) | (3 << 16) | (hl << 8))


def _same(a, b):
    a = np.ascontiguousarray(a, f32)
    b = np.ascontiguousarray(b, f32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _sig(x):
    return (f32(1) / (f32(1) + _O.expf(-np.asarray(x, f32)))).astype(f32)


_O = None


@pytest.fixture(scope="module", params=[16, 8], ids=["hashed", "dense"])
def frame(oracle, request):
    global _O
    _O = oracle
    return _Frame(oracle, request.param)


def _aux_is_mode0(out, m0):
    """Outputs 0-7 follow the geometry only; 8-13 (world position and
    appearance colour) are the grid path's."""
    assert _same(out["others"], m0["others"])
    assert _same(out["n_contrib"], m0["n_contrib"]) and _same(out["final_T"], m0["final_T"])


@pytest.mark.parametrize("mode", [8, 9, 10])
def test_gaussian_only_is_the_colour_path(frame, mode):
    out = frame.hsh(mode, 1)
    m0 = frame.mode0()
    _aux_is_mode0(out, m0)
    if mode == 8:
        rows = np.maximum(f32(0), np.minimum(f32(1), frame.raw + f32(0.5)))
    elif mode == 10:
        rows = _sig(frame.raw)
    else:
        rows = frame.sh
    assert _same(out["color"], frame.colour(rows)["color"])


def test_no_grid_level_is_gaussian_only(frame):
    """Without grid levels (bits 8-15 of the level 0) nothing is looked up:
    mode 10 with decompose 0 is sigmoid(raw + 0)."""
    assert _same(frame.hsh(10, 0, hl=0)["color"], frame.colour(_sig(frame.raw))["color"])


def test_mode9_adds_the_grid_to_the_dc_terms(frame):
    col = frame.colour(frame.sh)["color"]
    g = frame.mode0()["color"]
    assert np.abs(g).max() > 0
    out = frame.hsh(9, 0)
    dc = [0, 16, 32]
    rest = [c for c in range(48) if c not in dc]
    assert _same(out["color"][rest], col[rest])
    a = out["color"][dc].astype(np.float64)
    b = col[dc].astype(np.float64) + g.astype(np.float64)
    assert np.abs(a - b).max() <= TOL * np.abs(b).max()
    assert not np.allclose(a, col[dc])  # the grid changed them
    ngp = frame.hsh(9, 2)
    assert _same(ngp["color"][dc], g) and _same(ngp["color"][rest], col[rest])


def _single_hits(frame, out):
    """(pixel rows, cols, splat ids, alpha) of the pixels with exactly one hit."""
    W, H = frame.W, frame.H
    one = out["others"][7] == 1
    ys, xs = np.nonzero(one)
    gx = (W + 15) // 16
    tiles = (ys // 16) * gx + xs // 16
    ranges = frame.b["ranges"].reshape(-1, 2)
    last = out["n_contrib"][0][ys, xs].astype(np.int64)
    ids = frame.b["vals"][ranges[tiles, 0].astype(np.int64) + last - 1].astype(np.int64)
    return ys, xs, ids, out["others"][1][ys, xs].astype(np.float64)


@pytest.mark.parametrize("mode,dec", [(8, 0), (8, 2), (10, 0), (10, 2)])
def test_single_hit_closed_form(frame, mode, dec):
    out = frame.hsh(mode, dec)
    m0 = frame.mode0()
    _aux_is_mode0(out, m0)
    ys, xs, ids, alpha = _single_hits(frame, out)
    assert ys.size > 50
    h = m0["color"][:, ys, xs].astype(np.float64) / alpha  # [3, n]
    raw = frame.raw[ids].T.astype(np.float64)
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))
    if mode == 8:
        g = np.clip(raw + 0.5, 0.0, 1.0)
        f = sig(h) if dec == 2 else np.clip(g + sig(h), 0.0, 1.0)
    else:
        f = sig(h if dec == 2 else raw + h)
    got = out["color"][:, ys, xs].astype(np.float64)
    assert np.abs(got - f * alpha).max() <= TOL * np.abs(f * alpha).max()
    if dec == 0:  # both parts matter: neither alone reproduces the output
        only_g = frame.hsh(mode, 1)["color"][:, ys, xs]
        only_h = frame.hsh(mode, 2)["color"][:, ys, xs]
        assert not np.allclose(got, only_g) and not np.allclose(got, only_h)
