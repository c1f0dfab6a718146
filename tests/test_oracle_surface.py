"""Pins the oracle's surface-potential render modes 1 and 5
(CR/forward.cu:1825-1908) on its mode-0 grid path, colour path and
query_feature, which the golden vectors, closed forms and autograd tests pin.

Mode 5's colour channels (features 12-14 of each level at the splat centre,
the same for every pixel of the splat) are linear in the hits: the colour
path's render over those per-splat rows, bit for bit.  The potential channels
pass a ReLU per hit, so they are checked on pixels with a single hit, where
mode 0's render of the same grid is h * alpha: max(0, -(h . n) + b) * alpha
(mode 1, b the second grid at the centre) or max(0, -(h . n)) * alpha
(mode 5), relative 1e-5 (h comes back through a division).  Every mode keeps
mode 0's auxiliary outputs.
"""
import numpy as np
import pytest

from nest_splat.scene import get_spec, make_scene

f32 = np.float32
TOL = 1e-5


class _Frame:
    def __init__(self, oracle, F):
        spec = get_spec("cfg1", P=300, W=64, H=48, L=3, F=F, log2T=11, log_scale_mu=-2.2, name=f"surf{F}")
        sc = self.sc = make_scene(spec)
        self.O, self.F, self.L = oracle, F, spec.L
        cam = sc.cameras[0]
        self.W, self.H = cam.image_width, cam.image_height
        self.pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                                     cam.full_proj_transform, self.W, self.H)
        self.b = oracle.binning(self.pre, self.W, self.H)
        self.ap = sc.ap_level.reshape(-1).copy()
        self.ap[::4] = 2.0
        self.grid = oracle.make_grid(self.L, F, spec.S, spec.base_res, sc.offsets, sc.table, spec.gridrange,
                                     spec.contract)
        rng = np.random.default_rng(5)
        self.t2 = rng.uniform(-0.1, 0.1, ((1 << 11) * self.L, 4)).astype(f32)
        self.r2 = np.float32([-1.6, 1.4])
        self.grid2 = oracle.make_grid(self.L, 4, spec.S, spec.base_res, sc.offsets, self.t2, self.r2, spec.contract)

    def mode(self, m, second=True):
        C = (4 if m == 1 else 7) * self.L
        return self.O.render(self.pre, self.b, self.W, self.H, C, self.grid, homotrans=self.sc.homotrans,
                             ap_level=self.ap, render_mode=m, level=self.L,
                             grid2=(self.sc.offsets, self.t2, self.r2) if second else None)

    def mode0(self):
        return self.O.render(self.pre, self.b, self.W, self.H, self.L * self.F, self.grid,
                             homotrans=self.sc.homotrans, ap_level=self.ap)

    def centre(self, grid, F):
        H = self.sc.homotrans.reshape(-1, 16)
        out = np.zeros((H.shape[0], self.L * F), f32)
        for i in range(H.shape[0]):
            pk = np.float32([H[i, 3], H[i, 7], H[i, 11]])
            out[i] = self.O.query_feature(grid, pk, int(np.floor(self.ap[i])), self.L * F)
        return out


def _same(a, b):
    a = np.ascontiguousarray(a, f32)
    b = np.ascontiguousarray(b, f32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _single(fr, out):
    W = fr.W
    one = out["others"][7] == 1
    ys, xs = np.nonzero(one)
    gx = (W + 15) // 16
    tiles = (ys // 16) * gx + xs // 16
    ranges = fr.b["ranges"].reshape(-1, 2)
    ids = fr.b["vals"][ranges[tiles, 0].astype(np.int64) + out["n_contrib"][0][ys, xs].astype(np.int64) - 1]
    return ys, xs, ids.astype(np.int64), out["others"][1][ys, xs].astype(np.float64)


@pytest.mark.parametrize("F,m", [(12, 1), (15, 5)])
def test_surface_modes(oracle, F, m):
    fr = _Frame(oracle, F)
    out = fr.mode(m)
    m0 = fr.mode0()
    assert _same(out["others"], m0["others"]) and _same(out["n_contrib"], m0["n_contrib"])
    ys, xs, ids, alpha = _single(fr, out)
    assert ys.size > 30
    normal = fr.pre["normal_opacity"][ids, :3].astype(np.float64)
    per = 4 if m == 1 else 7
    b = fr.centre(fr.grid2, 4).astype(np.float64) if m == 1 else None
    for l in range(fr.L):
        for i in range(4):
            h = np.stack([m0["color"][l * F + 3 * i + k, ys, xs] for k in range(3)], 1).astype(np.float64) / alpha[:, None]
            dot = (h * normal).sum(1)
            v = np.maximum(0.0, -dot + (b[ids, l * 4 + i] if m == 1 else 0.0))
            got = out["color"][l * per + i, ys, xs].astype(np.float64)
            assert np.abs(got - v * alpha).max() <= TOL * max(np.abs(v * alpha).max(), 1e-3), (l, i)
    assert np.abs(out["color"][[l * per + i for l in range(fr.L) for i in range(4)]]).max() > 0
    if m == 5:
        rgb = fr.centre(fr.grid, 15)[:, [l * 15 + 12 + c for l in range(fr.L) for c in range(3)]]
        col = fr.colour_rgb = fr.O.render(fr.pre, fr.b, fr.W, fr.H, rgb.shape[1], None, colors=np.ascontiguousarray(rgb))
        chans = [l * 7 + 4 + c for l in range(fr.L) for c in range(3)]
        assert _same(out["color"][chans], col["color"])
        assert np.abs(col["color"]).max() > 0


def test_mode1_without_second_grid_is_the_relu_alone(oracle):
    fr = _Frame(oracle, 12)
    out = fr.mode(1, second=False)
    ys, xs, ids, alpha = _single(fr, out)
    m0 = fr.mode0()
    normal = fr.pre["normal_opacity"][ids, :3].astype(np.float64)
    for i in range(4):
        h = np.stack([m0["color"][3 * i + k, ys, xs] for k in range(3)], 1).astype(np.float64) / alpha[:, None]
        v = np.maximum(0.0, -(h * normal).sum(1)) * alpha
        assert np.abs(out["color"][i, ys, xs] - v).max() <= TOL * max(np.abs(v).max(), 1e-3)
