"""ctypes binding of libnest_splat.so (the C ABI declared in include/nest_splat.h).

Torch owns every device buffer; this module only passes raw pointers, sizes
and the current HIP stream.  There is no fallback: if the library is missing
every entry point raises.
"""
from __future__ import annotations

import ctypes as ct
import os
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnest_splat.so")

NEST_OK = 0
NEST_ERR_INVALID_ARGUMENT = -1
NEST_ERR_UNSUPPORTED = -2
NEST_ERR_WORKSPACE = -3
NEST_ERR_HIP = -4
NEST_ERR_OVERFLOW = -5

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
MAX_LEVELS = 32
MAX_CHANNELS = 128
OTHERS_CHANNELS = 14

ABI_VERSION = 17
SCAN_NOALLOC_MAX = 268431360
(GEOM_DEPTH, GEOM_XY, GEOM_TILES, GEOM_OFFSETS, GEOM_RECORDS, GEOM_RADII, GEOM_SCAN_TMP, GEOM_DEPTH_ORDER,
 GEOM_ORDER_OFFSETS, GEOM_ORDER_TMP, GEOM_RGB, GEOM_CLAMPED, GEOM_RECT, GEOM_ORDER_RECT) = range(14)
GEOM_FIELDS = 14
BIN_PAIR_TILES, BIN_PAIR_IDS, BIN_KEYS, BIN_VALS, BIN_SORT_TMP = range(5)
BIN_FIELDS = 5
IMG_RANGES, IMG_FINAL_T, IMG_N_CONTRIB, IMG_LEVELS, IMG_TILE_ORDER = range(5)
IMG_FIELDS = 5
BWD_DTRANSMAT, BWD_DHOMO, BWD_DNORMAL, BWD_DCOLORS, BWD_GRADSUM = range(5)
BWD_FIELDS = 5
STAGES = ("preprocess", "scan", "duplicate", "sort", "ranges", "render", "depth_order")


class RasterSettings(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("image_height", ct.c_int32), ("image_width", ct.c_int32),
                ("tanfovx", ct.c_float), ("tanfovy", ct.c_float), ("scale_modifier", ct.c_float),
                ("viewmatrix", ct.c_float * 16), ("projmatrix", ct.c_float * 16), ("campos", ct.c_float * 3),
                ("beta", ct.c_float), ("prefiltered", ct.c_int32), ("debug", ct.c_int32),
                ("if_contract", ct.c_int32), ("max_intersections", ct.c_uint32)]


class HashGrid(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("levels", ct.c_uint32), ("level_dim", ct.c_uint32),
                ("log2_scale", ct.c_float), ("base_resolution", ct.c_uint32), ("align_corners", ct.c_int32),
                ("interpolation", ct.c_int32), ("table_dtype", ct.c_int32), ("table", ct.c_void_p),
                ("table_rows", ct.c_int64), ("offsets", ct.c_int32 * (MAX_LEVELS + 1)),
                ("gridrange", ct.c_float * 2), ("render_mode", ct.c_int32), ("hybrid_levels", ct.c_uint32),
                ("total_levels", ct.c_uint32),
                ("active_levels", ct.c_uint32), ("decompose", ct.c_uint32), ("table2", ct.c_void_p),
                ("table2_rows", ct.c_int64), ("offsets2", ct.c_int32 * (MAX_LEVELS + 1)), ("gridrange2", ct.c_float * 2),
                ("rows2", ct.c_void_p)]


MODE_BASELINE = 0
MODE_SURFACE = 1
MODE_BASELINE_DOUBLE = 2
MODE_BASELINE_BLEND_DOUBLE = 3
MODE_SURFACE_RGB = 5
MODE_CAT = 4
MODE_ADAPTIVE = 6
MODE_ADAPTIVE_ADD = 7
MODE_HYBRID_SH = 8
MODE_HYBRID_SH_POST = 9
MODE_HYBRID_SH_RAW = 10
MODE_ADAPTIVE_CAT = 12
MODE_ADAPTIVE_CAT_FAST = 13
MODE_ADAPTIVE_ZERO = 14
MODE_INFERENCE = 0x100


class Splats(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("P", ct.c_int32), ("means3D", ct.c_void_p), ("scales", ct.c_void_p),
                ("rotations", ct.c_void_p), ("opacities", ct.c_void_p), ("homotrans", ct.c_void_p),
                ("ap_level", ct.c_void_p), ("colors_precomp", ct.c_void_p), ("shs", ct.c_void_p),
                ("sh_degree", ct.c_int32), ("sh_coeffs", ct.c_int32), ("shapes", ct.c_void_p),
                ("kernel_type", ct.c_int32), ("reserved", ct.c_int32)]


class FrameOutputs(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("channels", ct.c_int32), ("out_color", ct.c_void_p),
                ("out_others", ct.c_void_p), ("radii", ct.c_void_p), ("cover_pixels", ct.c_void_p),
                ("trans_avg", ct.c_void_p)]


class BackwardIO(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("channels", ct.c_int32), ("dL_dout_color", ct.c_void_p),
                ("dL_dout_others", ct.c_void_p), ("dL_dmeans3D", ct.c_void_p), ("dL_dmeans2D", ct.c_void_p),
                ("dL_dcolors", ct.c_void_p), ("dL_dopacity", ct.c_void_p), ("dL_dshs", ct.c_void_p),
                ("dL_dscales", ct.c_void_p), ("dL_drotations", ct.c_void_p), ("dL_dfeatures", ct.c_void_p),
                ("dL_dgradsum", ct.c_void_p), ("dL_dshapes", ct.c_void_p)]


class Timing(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("enabled", ct.c_int32), ("ms", ct.c_float * 7),
                ("events", ct.c_void_p * 14), ("recorded", ct.c_uint32)]


def new_timing(enabled: bool = True) -> Timing:
    t = Timing()
    t.struct_size = ct.sizeof(Timing)
    t.enabled = int(bool(enabled))
    return t


def timing_read(t: Timing) -> dict:
    check(lib().nest_timing_read(ct.byref(t)), "nest_timing_read")
    return {n: float(t.ms[i]) for i, n in enumerate(STAGES)}


def timing_release(t: Timing) -> None:
    check(lib().nest_timing_release(ct.byref(t)), "nest_timing_release")


class Mlp(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("in_features", ct.c_int32), ("width", ct.c_int32),
                ("dtype", ct.c_int32), ("w1", ct.c_void_p), ("w2", ct.c_void_p), ("w3", ct.c_void_p)]


class RvqAttr(ct.Structure):
    _fields_ = [("struct_size", ct.c_uint32), ("P", ct.c_int64), ("stages", ct.c_int32),
                ("codebook_size", ct.c_int32), ("dim", ct.c_int32), ("activation", ct.c_int32),
                ("codebooks", ct.c_void_p), ("indices", ct.c_void_p), ("bias", ct.POINTER(ct.c_float)),
                ("out", ct.c_void_p), ("raw_out", ct.c_void_p)]


RVQ_BATCH_MAX = 4

EXPORTS = {
    "nest_abi_version": (ct.c_int, []),
    "nest_last_error": (ct.c_char_p, []),
    "nest_geom_layout": (ct.c_int, [ct.c_int32, ct.POINTER(ct.c_size_t), ct.POINTER(ct.c_size_t)]),
    "nest_binning_layout": (ct.c_int, [ct.c_int64, ct.POINTER(ct.c_size_t), ct.POINTER(ct.c_size_t)]),
    "nest_image_layout": (ct.c_int, [ct.c_int32, ct.c_int32, ct.POINTER(ct.c_size_t), ct.POINTER(ct.c_size_t)]),
    "nest_hashgrid_levels": (ct.c_int, [ct.POINTER(HashGrid), ct.POINTER(ct.c_float), ct.POINTER(ct.c_uint32),
                                        ct.POINTER(ct.c_uint32)]),
    "nest_forward_geometry": (ct.c_int, [ct.POINTER(RasterSettings), ct.POINTER(Splats), ct.c_void_p, ct.c_size_t,
                                         ct.c_void_p, ct.POINTER(ct.c_int64), ct.POINTER(Timing), ct.c_void_p]),
    "nest_forward_render": (ct.c_int, [ct.POINTER(RasterSettings), ct.POINTER(HashGrid), ct.POINTER(Splats),
                                       ct.c_void_p, ct.c_size_t, ct.c_void_p, ct.c_size_t, ct.c_void_p, ct.c_size_t,
                                       ct.c_int64, ct.POINTER(FrameOutputs), ct.POINTER(Timing), ct.c_void_p]),
    "nest_binning_keys": (ct.c_int, [ct.c_int32, ct.c_int32, ct.c_int32, ct.c_void_p, ct.c_size_t, ct.c_void_p,
                                     ct.c_size_t, ct.c_void_p, ct.c_size_t, ct.c_int64, ct.c_void_p]),
    "nest_mark_visible": (ct.c_int, [ct.c_int32, ct.c_void_p, ct.POINTER(ct.c_float), ct.c_void_p, ct.c_void_p]),
    "nest_build_homotrans": (ct.c_int, [ct.c_int64, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p]),
    "nest_backward_layout": (ct.c_int, [ct.c_int32, ct.c_int32, ct.POINTER(ct.c_size_t), ct.POINTER(ct.c_size_t)]),
    "nest_backward": (ct.c_int, [ct.POINTER(RasterSettings), ct.POINTER(HashGrid), ct.POINTER(Splats), ct.c_void_p,
                                 ct.c_size_t, ct.c_void_p, ct.c_size_t, ct.c_void_p, ct.c_size_t, ct.c_int64,
                                 ct.POINTER(BackwardIO), ct.c_void_p, ct.c_size_t, ct.c_void_p]),
    "nest_timing_read": (ct.c_int, [ct.POINTER(Timing)]),
    "nest_timing_release": (ct.c_int, [ct.POINTER(Timing)]),
    "nest_scan_workspace_size": (ct.c_size_t, [ct.c_int64]),
    "nest_inclusive_scan_u32": (ct.c_int, [ct.c_void_p, ct.c_void_p, ct.c_int64, ct.c_void_p, ct.c_size_t,
                                           ct.c_void_p]),
    "nest_inclusive_scan_u32_noalloc": (ct.c_int, [ct.c_void_p, ct.c_void_p, ct.c_int64, ct.c_void_p]),
    "nest_sort_workspace_size": (ct.c_size_t, [ct.c_int64]),
    "nest_sort_pairs_u64": (ct.c_int, [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int64, ct.c_int32,
                                       ct.c_void_p, ct.c_size_t, ct.c_void_p]),
    "nest_grid_encode": (ct.c_int, [ct.c_void_p, ct.c_int64, ct.c_int32, ct.c_void_p, ct.c_int64, ct.c_int32,
                                    ct.POINTER(ct.c_int32), ct.c_int32, ct.c_int32, ct.c_float, ct.c_int32, ct.c_int32,
                                    ct.c_int32, ct.c_int32, ct.c_void_p, ct.c_void_p]),
    "nest_grid_encode_backward": (ct.c_int, [ct.c_void_p, ct.c_int64, ct.c_int32, ct.c_void_p, ct.c_int64, ct.c_int32,
                                             ct.POINTER(ct.c_int32), ct.c_int32, ct.c_int32, ct.c_float, ct.c_int32,
                                             ct.c_int32, ct.c_int32, ct.c_int32, ct.c_void_p, ct.c_void_p, ct.c_void_p,
                                             ct.c_void_p]),
    "nest_mlp_decode": (ct.c_int, [ct.POINTER(Mlp), ct.c_void_p, ct.c_int64, ct.c_int64, ct.c_int64, ct.c_int32,
                                   ct.c_void_p, ct.POINTER(ct.c_float), ct.c_void_p, ct.POINTER(ct.c_float),
                                   ct.c_void_p, ct.c_int64, ct.c_int64, ct.c_void_p]),
    "nest_rvq_decode": (ct.c_int, [ct.c_int64, ct.c_int32, ct.c_int32, ct.c_int32, ct.c_void_p, ct.c_void_p,
                                   ct.POINTER(ct.c_float), ct.c_int32, ct.c_void_p, ct.c_void_p, ct.c_void_p]),
    "nest_rvq_decode_batch": (ct.c_int, [ct.c_int32, ct.POINTER(RvqAttr), ct.c_void_p]),
}

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python nest-splatting_amd/build.py` "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = ct.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.nest_abi_version() != ABI_VERSION:
            raise RuntimeError("libnest_splat.so ABI version mismatch")
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc == NEST_OK:
        return
    msg = lib().nest_last_error().decode(errors="replace")
    if rc == NEST_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t: Optional[torch.Tensor]):
    if t is None or t.numel() == 0:
        return None
    return ct.c_void_p(t.data_ptr())


def stream_ptr(device=None):
    return ct.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def geom_layout(P: int):
    offs = (ct.c_size_t * GEOM_FIELDS)()
    tot = ct.c_size_t()
    check(lib().nest_geom_layout(P, offs, ct.byref(tot)), "nest_geom_layout")
    return list(offs), tot.value


def binning_layout(NR: int):
    offs = (ct.c_size_t * BIN_FIELDS)()
    tot = ct.c_size_t()
    check(lib().nest_binning_layout(NR, offs, ct.byref(tot)), "nest_binning_layout")
    return list(offs), tot.value


def image_layout(W: int, H: int):
    offs = (ct.c_size_t * IMG_FIELDS)()
    tot = ct.c_size_t()
    check(lib().nest_image_layout(W, H, offs, ct.byref(tot)), "nest_image_layout")
    return list(offs), tot.value


def hashgrid_levels(levels: int, level_dim: int, log2_scale: float, base_resolution: int, offsets,
                    align_corners: bool = False):
    """Per-level (scale, resolution, hashed) of a grid as the library's
    lookups use them (nest_hashgrid_levels; host-only)."""
    g = HashGrid()
    g.struct_size = ct.sizeof(HashGrid)
    g.levels, g.level_dim = int(levels), int(level_dim)
    g.log2_scale, g.base_resolution = float(log2_scale), int(base_resolution)
    g.align_corners = int(bool(align_corners))
    for i, o in enumerate(offsets):
        g.offsets[i] = int(o)
    g.table_rows = int(offsets[levels])
    sc = (ct.c_float * max(1, levels))()
    res = (ct.c_uint32 * max(1, levels))()
    hs = (ct.c_uint32 * max(1, levels))()
    check(lib().nest_hashgrid_levels(ct.byref(g), sc, res, hs), "nest_hashgrid_levels")
    return [float(v) for v in sc[:levels]], [int(v) for v in res[:levels]], [bool(v) for v in hs[:levels]]


def view(buf: torch.Tensor, offset: int, dtype: torch.dtype, shape) -> torch.Tensor:
    """A typed view into a uint8 workspace at a byte offset."""
    n = 1
    for s in shape:
        n *= s
    es = torch.empty((), dtype=dtype).element_size()
    return buf[offset: offset + n * es].view(dtype).view(*shape)
