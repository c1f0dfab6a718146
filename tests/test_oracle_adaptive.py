"""Pins the oracle's render mode 6 (adaptive, CR/forward.cu:1283-1325) on its
mode-0 grid path, its colour path and its mode 7, which the golden vectors,
the closed-form pins and the other mode tests pin.

A hit's feature at channel i < level*F is 0.5 * row[i] + 0.5 * grid[i], the
row being the splat's C floats and the grid its `level` levels at the hit;
the channels past level*F stay 0.  Halving is exact, so:
  - zero rows give half of mode 0's render, bit for bit;
  - a zero table gives half of the colour path's render over the rows'
    first level*F floats, bit for bit;
  - it is mode 7 with every row's weight 0.5, bit for bit (fmaf(0.5, r,
    0.5 * g) and 0.5 * r + 0.5 * g round the same exact sum);
  - the aux outputs (world position, appearance colour, contributors) are
    mode 0's.
"""
import numpy as np
import pytest

from nest_splat.scene import get_spec, make_scene

f32 = np.float32


class _Frame:
    def __init__(self, oracle, F, contract):
        spec = get_spec("cfg3" if contract else "cfg1", P=400, W=64, H=48, L=4, F=F, log2T=12, log_scale_mu=-2.2,
                        cam_dist=2.6, name=f"adaptive{F}{int(contract)}")
        sc = self.sc = make_scene(spec)
        self.O = oracle
        cam = sc.cameras[0]
        self.W, self.H = cam.image_width, cam.image_height
        self.pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                                     cam.full_proj_transform, self.W, self.H)
        self.b = oracle.binning(self.pre, self.W, self.H)
        assert self.b["num_rendered"] > 0
        self.L, self.F, self.spec = spec.L, F, spec
        self.ap = sc.ap_level.reshape(-1).copy()
        self.ap[::4] = 2.0  # some splats look up fewer levels
        self.grid = self.make_grid(sc.table)

    def make_grid(self, table):
        sp = self.spec
        return self.O.make_grid(self.L, self.F, sp.S, sp.base_res, self.sc.offsets, table, sp.gridrange, sp.contract)

    def rows(self, C, seed=5):
        return np.random.default_rng(seed).normal(0.0, 0.7, (self.sc.spec.P, C)).astype(f32)

    def mode6(self, rows, grid=None):
        return self.O.render(self.pre, self.b, self.W, self.H, rows.shape[1], grid or self.grid,
                             homotrans=self.sc.homotrans, ap_level=self.ap, colors=rows, render_mode=6, level=self.L)

    def mode0(self, C):
        return self.O.render(self.pre, self.b, self.W, self.H, C, self.grid, homotrans=self.sc.homotrans,
                             ap_level=self.ap)


def _same(a, b):
    a = np.ascontiguousarray(a, f32)
    b = np.ascontiguousarray(b, f32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module", params=[(4, False), (2, True), (8, False)], ids=["F4", "F2-contracted", "F8"])
def frame(oracle, request):
    return _Frame(oracle, *request.param)


@pytest.mark.parametrize("extra", [0, 3])
def test_zero_rows_are_half_the_grid_render(frame, extra):
    n = frame.L * frame.F
    out = frame.mode6(np.zeros((frame.sc.spec.P, n + extra), f32))
    m0 = frame.mode0(n)
    assert np.abs(m0["color"]).max() > 0
    assert _same(out["color"][:n], f32(0.5) * m0["color"])
    assert not out["color"][n:].any()
    assert _same(out["others"], m0["others"]) and _same(out["n_contrib"], m0["n_contrib"])
    assert _same(out["final_T"], m0["final_T"])


@pytest.mark.parametrize("extra", [0, 3])
def test_zero_table_is_half_the_colour_path(frame, extra):
    n = frame.L * frame.F
    rows = frame.rows(n + extra)
    out = frame.mode6(rows, frame.make_grid(np.zeros_like(frame.sc.table)))
    col = frame.O.render(frame.pre, frame.b, frame.W, frame.H, n, None, colors=np.ascontiguousarray(rows[:, :n]))
    assert np.abs(col["color"]).max() > 0
    assert _same(out["color"][:n], f32(0.5) * col["color"])
    assert not out["color"][n:].any()  # row entries past level*F are not read


def test_is_mode7_with_weight_half(frame):
    n = frame.L * frame.F
    rows = frame.rows(n + 2, seed=8)
    out = frame.mode6(rows)
    r7 = np.concatenate([rows[:, :n], np.full((rows.shape[0], 1), 0.5, f32)], axis=1)
    m7 = frame.O.render(frame.pre, frame.b, frame.W, frame.H, n, frame.grid, homotrans=frame.sc.homotrans,
                        ap_level=frame.ap, colors=r7, render_mode=7, level=(frame.L << 16) | (frame.L << 8))
    assert _same(out["color"][:n], m7["color"]) and _same(out["others"], m7["others"])
    # both halves matter
    m0 = frame.mode0(n)
    col = frame.O.render(frame.pre, frame.b, frame.W, frame.H, n, None, colors=np.ascontiguousarray(rows[:, :n]))
    assert not np.allclose(out["color"][:n], f32(0.5) * m0["color"])
    assert not np.allclose(out["color"][:n], f32(0.5) * col["color"])


def test_fewer_levels_than_the_grid(frame):
    """level below the grid's levels: only those levels are looked up and
    blended; the rest of the row is not read."""
    n1 = 2 * frame.F
    rows = frame.rows(frame.L * frame.F, seed=11)
    out = frame.O.render(frame.pre, frame.b, frame.W, frame.H, rows.shape[1], frame.grid,
                         homotrans=frame.sc.homotrans, ap_level=frame.ap, colors=rows, render_mode=6, level=2)
    r7 = np.concatenate([rows[:, :n1], np.full((rows.shape[0], 1), 0.5, f32)], axis=1)
    m7 = frame.O.render(frame.pre, frame.b, frame.W, frame.H, n1, frame.grid, homotrans=frame.sc.homotrans,
                        ap_level=frame.ap, colors=r7, render_mode=7, level=(2 << 16) | (2 << 8))
    assert _same(out["color"][:n1], m7["color"]) and not out["color"][n1:].any()
