"""Pins the oracle's dual-grid render modes 2 (baseline_double) and 3
(baseline_blend_double) (CR/forward.cu:1146-1217, :1975-2004) on its mode-0
grid path, its colour path and its query_feature, which the golden vectors,
the closed-form pins and the autograd tests pin.

A hit's features in mode 2 are the first grid's at the hit followed by the
second grid's at the splat centre, which is the same for every pixel of the
splat: so the first half of the channels is mode 0's render, bit for bit, and
the second half the colour path's render over per-splat rows of the second
grid's features at the centres.  Mode 3 blends only those rows, then adds the
first grid's features at the pixel's blended position with the appearance
level of its tile's first splat: the colour path's render plus one
query_feature per pixel, bit for bit.
"""
import numpy as np
import pytest

from nest_splat.scene import get_spec, make_scene

f32 = np.float32


class _Frame:
    def __init__(self, oracle, contract):
        spec = get_spec("cfg3" if contract else "cfg1", P=400, W=64, H=48, L=4, F=4, log2T=12, log_scale_mu=-2.2,
                        cam_dist=2.6, name=f"dual{int(contract)}")
        sc = self.sc = make_scene(spec)
        self.O = oracle
        cam = sc.cameras[0]
        self.W, self.H = cam.image_width, cam.image_height
        self.pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                                     cam.full_proj_transform, self.W, self.H)
        self.b = oracle.binning(self.pre, self.W, self.H)
        assert self.b["num_rendered"] > 0
        self.L, self.F = spec.L, spec.F
        rng = np.random.default_rng(9)
        self.table2 = rng.uniform(-0.2, 0.2, sc.table.shape).astype(f32)
        self.range2 = np.float32([spec.gridrange[0] * 1.2, spec.gridrange[1] * 0.9])
        self.ap = sc.ap_level.reshape(-1).copy()
        self.ap[::4] = 2.0  # some splats query fewer levels
        self.grid1 = oracle.make_grid(self.L, self.F, spec.S, spec.base_res, sc.offsets, sc.table, spec.gridrange,
                                      spec.contract)
        self.grid2 = oracle.make_grid(self.L, self.F, spec.S, spec.base_res, sc.offsets, self.table2, self.range2,
                                      spec.contract)

    def render(self, mode, with_grid2=True):
        g2 = (self.sc.offsets, self.table2, self.range2) if with_grid2 else None
        C = (2 if mode == 2 else 1) * self.L * self.F
        return self.O.render(self.pre, self.b, self.W, self.H, C, self.grid1, homotrans=self.sc.homotrans,
                             ap_level=self.ap, render_mode=mode, level=self.L, grid2=g2)

    def mode0(self):
        return self.O.render(self.pre, self.b, self.W, self.H, self.L * self.F, self.grid1,
                             homotrans=self.sc.homotrans, ap_level=self.ap)

    def centre_rows(self):
        H = self.sc.homotrans.reshape(-1, 16)
        rows = np.zeros((H.shape[0], self.L * self.F), f32)
        for i in range(H.shape[0]):
            pk = np.float32([H[i, 3], H[i, 7], H[i, 11]])
            rows[i] = self.O.query_feature(self.grid2, pk, int(np.floor(self.ap[i])), self.L * self.F)
        return rows

    def colour(self, rows):
        return self.O.render(self.pre, self.b, self.W, self.H, rows.shape[1], None, colors=np.ascontiguousarray(rows))


def _same(a, b):
    a = np.ascontiguousarray(a, f32)
    b = np.ascontiguousarray(b, f32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module", params=[False, True], ids=["affine", "contracted"])
def frame(oracle, request):
    return _Frame(oracle, request.param)


def test_mode2_is_mode0_then_the_centre_rows(frame):
    out = frame.render(2)
    m0 = frame.mode0()
    n = frame.L * frame.F
    rows = frame.centre_rows()
    assert np.abs(rows).max() > 0
    assert _same(out["color"][:n], m0["color"])
    assert _same(out["color"][n:], frame.colour(rows)["color"])
    assert _same(out["others"], m0["others"]) and _same(out["n_contrib"], m0["n_contrib"])


def test_mode2_without_second_grid(frame):
    out = frame.render(2, with_grid2=False)
    n = frame.L * frame.F
    assert _same(out["color"][:n], frame.mode0()["color"]) and not out["color"][n:].any()


def _spatial(frame, out):
    """The per-pixel query after the loop: the first grid at the blended
    position, appearance level of the tile's first splat (0 without hits)."""
    W, H, n = frame.W, frame.H, frame.L * frame.F
    gx = (W + 15) // 16
    ranges = frame.b["ranges"].reshape(-1, 2)
    vals = frame.b["vals"]
    fs = np.zeros((n, H, W), f32)
    for y in range(H):
        for x in range(W):
            tile = (y // 16) * gx + x // 16
            pap = 0
            if out["n_contrib"][0, y, x] > 0:
                pap = int(np.floor(frame.ap[vals[ranges[tile, 0]]]))
            pos = np.float32(out["others"][8:11, y, x])
            fs[:, y, x] = frame.O.query_feature(frame.grid1, pos, pap, n)
    return fs


@pytest.mark.parametrize("with_grid2", [True, False])
def test_mode3_is_the_centre_rows_plus_the_spatial_query(frame, with_grid2):
    out = frame.render(3, with_grid2)
    m0 = frame.mode0()
    rows = frame.centre_rows() if with_grid2 else np.zeros((frame.sc.spec.P, frame.L * frame.F), f32)
    fs = _spatial(frame, out)
    assert np.abs(fs).max() > 0
    assert _same(out["color"], frame.colour(rows)["color"] + fs)
    assert _same(out["others"], m0["others"])
