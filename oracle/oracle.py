"""ctypes front end of the CPU oracle (oracle/nest_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  All functions take
and return numpy arrays.  See nest_oracle.c for the floating-point contract
and the reference file:line each routine follows.
"""
from __future__ import annotations

import ctypes as ct
import math
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnest_oracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class OrGrid(ct.Structure):
    _fields_ = [("L", ct.c_int), ("F", ct.c_int), ("S", ct.c_float), ("H", ct.c_int),
                ("align_corners", ct.c_int), ("interp", ct.c_int), ("contract", ct.c_int),
                ("vmin", ct.c_float), ("vmax", ct.c_float),
                ("offsets", ct.c_void_p), ("table", ct.c_void_p), ("half_table", ct.c_int)]


class OrRenderArgs(ct.Structure):
    _fields_ = [("W", ct.c_int), ("H", ct.c_int), ("C", ct.c_int), ("level", ct.c_int),
                ("beta", ct.c_float), ("max_intersections", ct.c_uint32),
                ("ranges", ct.c_void_p), ("point_list", ct.c_void_p), ("xy", ct.c_void_p),
                ("transmat", ct.c_void_p), ("normal_opacity", ct.c_void_p), ("homotrans", ct.c_void_p),
                ("ap_level", ct.c_void_p), ("colors", ct.c_void_p), ("grid", OrGrid),
                ("out_color", ct.c_void_p), ("out_others", ct.c_void_p), ("final_T", ct.c_void_p),
                ("n_contrib", ct.c_void_p), ("render_mode", ct.c_int), ("cover_pixels", ct.c_void_p),
                ("trans_avg", ct.c_void_p), ("shapes", ct.c_void_p), ("kernel_type", ct.c_int),
                ("offsets2", ct.c_void_p), ("table2", ct.c_void_p), ("vmin2", ct.c_float), ("vmax2", ct.c_float)]


class OrRenderBwdArgs(ct.Structure):
    _fields_ = [("W", ct.c_int), ("H", ct.c_int), ("C", ct.c_int), ("level", ct.c_int), ("beta", ct.c_float),
                ("ranges", ct.c_void_p), ("point_list", ct.c_void_p), ("xy", ct.c_void_p),
                ("transmat", ct.c_void_p), ("normal_opacity", ct.c_void_p), ("homotrans", ct.c_void_p),
                ("ap_level", ct.c_void_p), ("colors", ct.c_void_p), ("grid", OrGrid),
                ("final_T", ct.c_void_p), ("n_contrib", ct.c_void_p), ("dL_dpix", ct.c_void_p),
                ("dL_dothers", ct.c_void_p), ("dtable", ct.c_void_p), ("dtransmat", ct.c_void_p),
                ("dhomo", ct.c_void_p), ("dmean2D", ct.c_void_p), ("dnormal", ct.c_void_p),
                ("dopacity", ct.c_void_p), ("dcolors", ct.c_void_p), ("gradsum", ct.c_void_p),
                ("render_mode", ct.c_int), ("shapes", ct.c_void_p), ("kernel_type", ct.c_int),
                ("dshapes", ct.c_void_p)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ct.CDLL(_LIB_PATH)
        L.or_expf.restype = ct.c_float
        L.or_expf.argtypes = [ct.c_float]
        L.or_expf_n.argtypes = [ct.c_int, f32p, f32p]
        L.or_logf.restype = ct.c_float
        L.or_logf.argtypes = [ct.c_float]
        L.or_powf.restype = ct.c_float
        L.or_powf.argtypes = [ct.c_float, ct.c_float]
        L.or_logf_n.argtypes = [ct.c_int, f32p, f32p]
        L.or_powf_n.argtypes = [ct.c_int, f32p, f32p, f32p]
        L.or_round_bf16.restype = ct.c_float
        L.or_round_bf16.argtypes = [ct.c_float]
        L.or_round_f16.restype = ct.c_float
        L.or_round_f16.argtypes = [ct.c_float]
        L.or_higher_msb.restype = ct.c_uint32
        L.or_higher_msb.argtypes = [ct.c_uint32]
        L.or_preprocess.argtypes = [ct.c_int, f32p, f32p, f32p, f32p, ct.c_float, f32p, f32p,
                                    ct.c_int, ct.c_int, i32p, f32p, f32p, f32p, f32p, u32p]
        L.or_inclusive_scan_u32.argtypes = [ct.c_int, u32p, u32p]
        L.or_duplicate_keys.argtypes = [ct.c_int, f32p, f32p, i32p, u32p, ct.c_uint32, ct.c_uint32, u64p, u32p]
        L.or_sort_pairs.argtypes = [ct.c_int, u64p, u32p]
        L.or_tile_ranges.argtypes = [ct.c_int, u64p, ct.c_int, u32p]
        L.or_render.argtypes = [ct.POINTER(OrRenderArgs), ct.c_int, ct.c_int, ct.c_int]
        L.or_query_feature.argtypes = [ct.POINTER(OrGrid), f32p, ct.c_uint32, ct.c_int, f32p]
        L.or_grid_normalise.argtypes = [ct.POINTER(OrGrid), f32p, f32p]
        L.or_grid_normalise.restype = ct.c_int
        L.or_grid_encode.argtypes = [ct.POINTER(OrGrid), ct.c_int, f32p, f32p]
        L.or_level_scale.argtypes = [ct.c_float, ct.c_int, ct.c_int, ct.POINTER(ct.c_float), ct.POINTER(ct.c_uint32)]
        L.or_mlp.argtypes = [ct.c_int, ct.c_int, f32p, f32p, ct.c_void_p, f32p, f32p, f32p, ct.c_int, ct.c_int,
                             ct.c_void_p, f32p, ct.c_int]
        L.or_sh16.argtypes = [f32p, f32p]
        L.or_rvq_decode.argtypes = [ct.c_int, ct.c_int, ct.c_int, ct.c_int, f32p, u16p, ct.c_void_p, f32p]
        L.or_activate.argtypes = [ct.c_int, f32p, f32p, f32p, f32p, f32p, f32p]
        L.or_render_backward.argtypes = [ct.POINTER(OrRenderBwdArgs)]
        L.or_preprocess_backward.argtypes = [ct.c_int, f32p, f32p, f32p, i32p, f32p, f32p, f32p, ct.c_int, ct.c_int,
                                             ct.c_void_p, ct.c_int, ct.c_int, f32p, ct.c_void_p, ct.c_void_p, f32p,
                                             f32p, f32p, f32p, f32p, f32p, f32p, ct.c_void_p]
        L.or_grid_encode_backward.argtypes = [ct.POINTER(OrGrid), ct.c_int, f32p, f32p, f32p, ct.c_void_p]
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        L.or_sh_colors.argtypes = [ct.c_int, ct.c_int, ct.c_int, f32p, f32p, f32p, i32p, f32p, u8p]
        L.or_mark_visible.argtypes = [ct.c_int, f32p, f32p, u8p]
        L.or_max_threads.restype = ct.c_int
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def expf(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_expf_n(x.size, x.reshape(-1), y.reshape(-1))
    return y


def logf(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_logf_n(x.size, x.reshape(-1), y.reshape(-1))
    return y


def powf(x, e) -> np.ndarray:
    x, e = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(e, np.float32))
    x, e = np.ascontiguousarray(x), np.ascontiguousarray(e)
    y = np.empty_like(x)
    lib().or_powf_n(x.size, x.reshape(-1), e.reshape(-1), y.reshape(-1))
    return y


def round_bf16(x):
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x7FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, (u | 0x400000).astype(np.uint32), r)
    return r.view(np.float32)


def higher_msb(n: int) -> int:
    return int(lib().or_higher_msb(n))


def level_scale(S: float, H: int, l: int):
    sc = ct.c_float()
    res = ct.c_uint32()
    lib().or_level_scale(ct.c_float(S), H, l, ct.byref(sc), ct.byref(res))
    return sc.value, res.value


def sh_colors(pre, means, campos, shs, deg):
    """computeColorFromSH for the splats preprocess kept (radii > 0): returns
    (rgb [P,3], clamped [P,3] uint8); other rows stay 0."""
    P = means.shape[0]
    shs = _c(shs, np.float32).reshape(P, -1, 3)
    rgb = np.zeros((P, 3), np.float32)
    clamped = np.zeros((P, 3), np.uint8)
    lib().or_sh_colors(P, int(deg), shs.shape[1], _c(means, np.float32), _c(campos, np.float32).reshape(-1),
                       shs, _c(pre["radii"], np.int32), rgb, clamped)
    return rgb, clamped


def mark_visible(means, view):
    P = means.shape[0]
    out = np.zeros(P, np.uint8)
    lib().or_mark_visible(P, _c(means, np.float32), _c(view, np.float32).reshape(-1), out)
    return out.astype(bool)


def preprocess(means, scales, rots, opac, view, proj, W, H, scale_mod=1.0):
    P = means.shape[0]
    out = dict(radii=np.zeros(P, np.int32), xy=np.zeros((P, 2), np.float32),
               depth=np.zeros(P, np.float32), transmat=np.zeros((P, 9), np.float32),
               normal_opacity=np.zeros((P, 4), np.float32), tiles=np.zeros(P, np.uint32))
    lib().or_preprocess(P, _c(means, np.float32), _c(scales, np.float32), _c(rots, np.float32),
                        _c(opac, np.float32).reshape(-1), float(scale_mod),
                        _c(view, np.float32).reshape(-1), _c(proj, np.float32).reshape(-1), W, H,
                        out["radii"], out["xy"], out["depth"], out["transmat"], out["normal_opacity"], out["tiles"])
    return out


def binning(pre: dict, W: int, H: int):
    """scan -> duplicate -> stable sort -> tile ranges (rasterizer_impl.cu:355-396)."""
    P = pre["radii"].shape[0]
    gx, gy = (W + 15) // 16, (H + 15) // 16
    offs = np.zeros(P, np.uint32)
    if P:
        lib().or_inclusive_scan_u32(P, _c(pre["tiles"], np.uint32), offs)
    NR = int(offs[-1]) if P else 0
    keys = np.zeros(max(NR, 1), np.uint64)
    vals = np.zeros(max(NR, 1), np.uint32)
    lib().or_duplicate_keys(P, pre["xy"], pre["depth"], pre["radii"], offs, gx, gy, keys, vals)
    keys_unsorted, vals_unsorted = keys[:NR].copy(), vals[:NR].copy()
    lib().or_sort_pairs(NR, keys, vals)
    ranges = np.zeros((gx * gy, 2), np.uint32)
    lib().or_tile_ranges(NR, keys, gx * gy, ranges)
    return dict(offsets=offs, num_rendered=NR, keys_unsorted=keys_unsorted, vals_unsorted=vals_unsorted,
                keys=keys[:NR], vals=vals[:NR], ranges=ranges)


def make_grid(L, F, S, H, offsets, table, gridrange, contract=False, align_corners=False, interp=0):
    offsets = _c(offsets, np.int32)
    half = table.dtype == np.float16
    table = np.ascontiguousarray(table)
    g = OrGrid(L, F, S, H, int(align_corners), int(interp), int(contract),
               float(gridrange[0]), float(gridrange[1]),
               offsets.ctypes.data, table.ctypes.data, int(half))
    g._keep = (offsets, table)
    return g


def render(pre, binres, W, H, C, grid: Optional[OrGrid], homotrans=None, ap_level=None, colors=None,
           beta=0.0, max_intersections=0, row_stride=1, row_phase=0, threads=0, render_mode=0, level=None,
           record_transmittance=False, shapes=None, kernel_type=0, grid2=None):
    """renderCUDAsurfelForward for every pixel.  render_mode 0 (grid levels
    grid.L, or the colour path without a grid), 4, 7, 12, 13 or 14 (bit 8:
    inference); for modes 4, 7, 12, 13 and 14, level is the reference's packed level argument
    (total << 16 | hash levels << 8 | per-splat levels) and colors the
    per-splat feature rows; for modes 8, 9 and 10 (hybrid SH) level is
    decompose << 24 | SH degree << 16 | grid levels << 8, colors the rows of
    3 raw SH colours (8, 10) or 48 SH coefficients (9) and the grid one level
    of 3 channels.  record_transmittance adds cover_pixels and
    trans_avg ([P] each) to the result.  kernel_type 1-3 take the per-splat
    parameter from shapes [P].  Render modes 2 and 3 (level = the grids'
    levels, F = 4) take the second grid as grid2 = (offsets, float32 table,
    gridrange), or None for a missing one.  Render mode 6 (adaptive): level =
    the grid levels, colors rows of C floats."""
    HW = W * H
    out = dict(color=np.zeros((C, H, W), np.float32), others=np.zeros((14, H, W), np.float32),
               final_T=np.zeros((3, H, W), np.float32), n_contrib=np.zeros((2, H, W), np.uint32))
    if record_transmittance:
        P = len(pre["radii"])
        out["cover_pixels"] = np.zeros(P, np.float32)
        out["trans_avg"] = np.zeros(P, np.float32)
    keep = []

    def ptr(a, dt):
        if a is None:
            return None
        a = _c(a, dt)
        keep.append(a)
        return a.ctypes.data

    args = OrRenderArgs()
    args.W, args.H, args.C = W, H, C
    args.level = (0 if grid is None else grid.L) if level is None else level
    args.render_mode = render_mode
    args.beta = beta
    args.max_intersections = max_intersections
    args.ranges = ptr(binres["ranges"], np.uint32)
    args.point_list = ptr(binres["vals"] if binres["num_rendered"] else np.zeros(1, np.uint32), np.uint32)
    args.xy = ptr(pre["xy"], np.float32)
    args.transmat = ptr(pre["transmat"], np.float32)
    args.normal_opacity = ptr(pre["normal_opacity"], np.float32)
    args.homotrans = ptr(homotrans, np.float32)
    args.ap_level = ptr(ap_level, np.float32)
    args.colors = ptr(colors, np.float32)
    if grid is not None:
        args.grid = grid
    args.out_color = out["color"].ctypes.data
    args.out_others = out["others"].ctypes.data
    args.final_T = out["final_T"].ctypes.data
    args.n_contrib = out["n_contrib"].ctypes.data
    if record_transmittance:
        args.cover_pixels = out["cover_pixels"].ctypes.data
        args.trans_avg = out["trans_avg"].ctypes.data
    args.kernel_type = kernel_type
    if kernel_type != 0:
        args.shapes = ptr(np.asarray(shapes, np.float32).reshape(-1), np.float32)
    if grid2 is not None:
        args.offsets2 = ptr(grid2[0], np.int32)
        args.table2 = ptr(grid2[1], np.float32)
        args.vmin2, args.vmax2 = float(grid2[2][0]), float(grid2[2][1])
    lib().or_render(ct.byref(args), row_stride, row_phase, threads)
    return out


def render_backward(pre, binres, fwd, W, H, C, grid: Optional[OrGrid], dL_dpix, dL_dothers, homotrans=None,
                    ap_level=None, colors=None, beta=0.0, render_mode=0, level=None, shapes=None, kernel_type=0):
    """renderCUDAsurfelBackward (modes 0, 4, 7, 12 and 14) for every pixel, given the
    forward's final_T / n_contrib (fwd = render(...)'s result).  Returns the
    per-splat gradients (dtransmat [P,9], dhomo [P,9], dmean2D [P,3],
    dnormal [P,3], dopacity [P], dcolors [P,C], or [P,hyb*F] in mode 4,
    [P,total*F+1] in modes 7 and 12, [P,hyb*F+1] in mode 14, gradsum [P])
    and dtable [rows, F]; kernel_type 1-3 (with shapes [P]) adds dshapes [P].
    Modes 4, 7, 12 and 14 take the packed level
    (total << 16) | (active grid levels << 8) | per-splat levels and the
    per-splat rows as colors."""
    P = pre["radii"].shape[0]
    rows = 0 if grid is None else grid._keep[1].shape[0]
    F = 1 if grid is None else grid.F
    if render_mode not in (0, 4, 7, 12, 14) or (render_mode != 0 and (grid is None or level is None)):
        raise ValueError(f"render_backward: render_mode {render_mode} needs mode 0, or mode 4, 7, 12 or 14 with a grid "
                         f"and level")
    if render_mode == 0:
        dcol = C
    elif render_mode == 4:
        dcol = (level & 0xFF) * F
    elif render_mode == 14:
        dcol = (level & 0xFF) * F + 1
    else:
        dcol = ((level >> 16) & 0xFF) * F + 1
    out = dict(dtransmat=np.zeros((P, 9), np.float32), dhomo=np.zeros((P, 9), np.float32),
               dmean2D=np.zeros((P, 3), np.float32), dnormal=np.zeros((P, 3), np.float32),
               dopacity=np.zeros(P, np.float32), dcolors=np.zeros((P, max(dcol, 1)), np.float32),
               gradsum=np.zeros(P, np.float32), dtable=np.zeros((max(rows, 1), F), np.float32),
               dshapes=np.zeros(P, np.float32))
    keep = []

    def ptr(a, dt):
        if a is None:
            return None
        a = _c(a, dt)
        keep.append(a)
        return a.ctypes.data

    a = OrRenderBwdArgs()
    a.W, a.H, a.C = W, H, C
    a.level = (0 if grid is None else grid.L) if render_mode == 0 else level
    a.render_mode = render_mode
    a.beta = beta
    a.ranges = ptr(binres["ranges"], np.uint32)
    a.point_list = ptr(binres["vals"] if binres["num_rendered"] else np.zeros(1, np.uint32), np.uint32)
    a.xy = ptr(pre["xy"], np.float32)
    a.transmat = ptr(pre["transmat"], np.float32)
    a.normal_opacity = ptr(pre["normal_opacity"], np.float32)
    a.homotrans = ptr(homotrans, np.float32)
    a.ap_level = ptr(ap_level, np.float32)
    a.colors = ptr(colors, np.float32)
    if grid is not None:
        a.grid = grid
    a.final_T = ptr(fwd["final_T"], np.float32)
    a.n_contrib = ptr(fwd["n_contrib"], np.uint32)
    a.dL_dpix = ptr(dL_dpix, np.float32)
    a.dL_dothers = ptr(dL_dothers, np.float32)
    for k in ("dtable", "dtransmat", "dhomo", "dmean2D", "dnormal", "dopacity", "dcolors", "gradsum", "dshapes"):
        setattr(a, k, out[k].ctypes.data)
    if kernel_type not in (0, 1, 2, 3) or (kernel_type != 0 and shapes is None):
        raise ValueError(f"render_backward: kernel_type {kernel_type} needs 0-3, with shapes for 1-3")
    a.kernel_type = kernel_type
    if kernel_type != 0:
        a.shapes = ptr(np.asarray(shapes, np.float32).reshape(-1), np.float32)
    lib().or_render_backward(ct.byref(a))
    if rows == 0:
        out["dtable"] = np.zeros((0, F), np.float32)
    out["dcolors"] = out["dcolors"][:, :dcol]
    return out


def preprocess_backward(means, scales, rots, radii, transmat, view, proj, W, H, dtransmat, dhomo, dnormal, dmean2D,
                        shs=None, sh_degree=0, campos=(0.0, 0.0, 0.0), clamped=None, dcolors=None):
    """preprocessCUDA backward: returns dmeans [P,3], dscales [P,2], drots [P,4],
    dmean2D [P,3] (the densification statistic) and dshs [P,M,3]."""
    P = means.shape[0]
    dm2 = _c(dmean2D, np.float32).copy()
    out = dict(dmeans=np.zeros((P, 3), np.float32), dscales=np.zeros((P, 2), np.float32),
               drots=np.zeros((P, 4), np.float32))
    M = 0
    sh_arr = None
    if shs is not None:
        sh_arr = _c(shs, np.float32).reshape(P, -1, 3)
        M = sh_arr.shape[1]
    dshs = np.zeros((P, max(M, 1), 3), np.float32)
    cl = None if clamped is None else _c(clamped, np.uint8)
    dc = None if dcolors is None else _c(dcolors, np.float32)
    lib().or_preprocess_backward(P, _c(means, np.float32), _c(scales, np.float32), _c(rots, np.float32),
                                 _c(radii, np.int32), _c(transmat, np.float32), _c(view, np.float32).reshape(-1),
                                 _c(proj, np.float32).reshape(-1), W, H,
                                 None if sh_arr is None else sh_arr.ctypes.data, int(sh_degree), M,
                                 _c(campos, np.float32).reshape(-1), None if cl is None else cl.ctypes.data,
                                 None if dc is None else dc.ctypes.data, _c(dtransmat, np.float32),
                                 _c(dhomo, np.float32), _c(dnormal, np.float32), dm2, out["dmeans"],
                                 out["dscales"], out["drots"], dshs.ctypes.data)
    out["dmean2D"] = dm2
    out["dshs"] = dshs[:, :M]
    return out


def grid_encode_backward(grid: OrGrid, inputs, grad, with_inputs=True):
    """GridEncoder backward: (grad_table [rows, F], grad_inputs [B,3] or None);
    grad is the forward output's gradient [B, L*F]."""
    inputs = _c(inputs, np.float32)
    B = inputs.shape[0]
    rows = grid._keep[1].shape[0]
    gt = np.zeros((rows, grid.F), np.float32)
    gi = np.zeros((B, 3), np.float32) if with_inputs else None
    lib().or_grid_encode_backward(ct.byref(grid), B, inputs, _c(grad, np.float32), gt,
                                  None if gi is None else gi.ctypes.data)
    return gt, gi


def query_feature(grid: OrGrid, xyz, ap, C):
    feat = np.zeros(C, np.float32)
    lib().or_query_feature(ct.byref(grid), _c(xyz, np.float32), int(ap), C, feat)
    return feat


def grid_normalise(grid: OrGrid, xyz):
    u = np.zeros(3, np.float32)
    oob = lib().or_grid_normalise(ct.byref(grid), _c(xyz, np.float32), u)
    return u, bool(oob)


def grid_encode(grid: OrGrid, inputs):
    inputs = _c(inputs, np.float32)
    B = inputs.shape[0]
    out = np.zeros((B, grid.L * grid.F), np.float32)
    lib().or_grid_encode(ct.byref(grid), B, inputs, out)
    return out


def sh16(u):
    o = np.zeros(16, np.float32)
    lib().or_sh16(_c(u, np.float32), o)
    return o


DTYPES = {"f32": 0, "f16": 1, "bf16": 2}


def mlp(feat_cm, dirs, alpha, W1, W2, W3, dtype="f32", bg=None, threads=0):
    """feat_cm: [C, npix] channel-major; dirs: [npix, 3] unit; returns [3, npix].
    threads: OpenMP threads over pixels (0 = the runtime default)."""
    C, npix = feat_cm.shape
    out = np.zeros((3, npix), np.float32)
    a = None if alpha is None else _c(alpha, np.float32).reshape(-1)
    b = None if bg is None else _c(bg, np.float32)
    lib().or_mlp(npix, C, _c(feat_cm, np.float32), _c(dirs, np.float32),
                 None if a is None else a.ctypes.data, _c(W1, np.float32), _c(W2, np.float32),
                 _c(W3, np.float32), W1.shape[0], DTYPES[dtype], None if b is None else b.ctypes.data, out,
                 int(threads))
    return out


def rvq_decode(cb, idx, bias=None):
    S, K, dim = cb.shape
    P = idx.shape[0]
    out = np.zeros((P, dim), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().or_rvq_decode(P, S, K, dim, _c(cb, np.float32), _c(idx, np.uint16),
                        None if b is None else b.ctypes.data, out)
    return out


def activate(sc_raw, rot_raw, op_raw):
    P = sc_raw.shape[0]
    sc = np.zeros((P, 2), np.float32)
    rot = np.zeros((P, 4), np.float32)
    op = np.zeros(P, np.float32)
    lib().or_activate(P, _c(sc_raw, np.float32), _c(rot_raw, np.float32), _c(op_raw, np.float32).reshape(-1),
                      sc, rot, op)
    return sc, rot, op


def ray_dirs(cam) -> np.ndarray:
    """Unit view directions per pixel, row-major [H*W, 3] (point_utils.py:31-46
    then torch_F.normalize), evaluated in float64 from the float32 camera."""
    W, H = cam.image_width, cam.image_height
    wv = cam.world_view_transform.astype(np.float64)
    c2w = np.linalg.inv(wv.T)
    ndc2pix = np.array([[W / 2, 0, 0, W / 2], [0, H / 2, 0, H / 2], [0, 0, 0, 1]], dtype=np.float64).T
    intr = ((c2w.T @ cam.full_proj_transform.astype(np.float64)) @ ndc2pix)[:3, :3].T
    gx, gy = np.meshgrid(np.arange(W, dtype=np.float64), np.arange(H, dtype=np.float64), indexing="xy")
    pts = np.stack([gx, gy, np.ones_like(gx)], -1).reshape(-1, 3)
    d = pts @ np.linalg.inv(intr).T @ c2w[:3, :3].T
    d = d / np.maximum(np.linalg.norm(d, axis=1, keepdims=True), 1e-12)
    return d.astype(np.float32)


def render_scene(scene, cam_index=0, row_stride=1, row_phase=0, threads=0, with_mlp=True):
    """Full oracle forward of one camera: preprocess, binning, render, MLP."""
    sp = scene.spec
    cam = scene.cameras[cam_index]
    W, H = cam.image_width, cam.image_height
    pre = preprocess(scene.means, scene.scales, scene.rotations, scene.opacity, cam.world_view_transform,
                     cam.full_proj_transform, W, H)
    b = binning(pre, W, H)
    grid = make_grid(sp.L, sp.F, sp.S, sp.base_res, scene.offsets, scene.table, sp.gridrange, sp.contract)
    r = render(pre, b, W, H, sp.C, grid, homotrans=scene.homotrans, ap_level=scene.ap_level,
               row_stride=row_stride, row_phase=row_phase, threads=threads)
    out = dict(pre=pre, bin=b, **r)
    if with_mlp:
        dirs = ray_dirs(cam)
        feat = r["color"].reshape(sp.C, -1)
        alpha = r["others"][1].reshape(-1)
        rgb = mlp(feat, dirs, alpha, scene.W1, scene.W2, scene.W3, sp.mlp_dtype, np.asarray(sp.bg, np.float32))
        out["rgb"] = rgb.reshape(3, H, W)
    return out


def max_threads() -> int:
    return int(lib().or_max_threads())
