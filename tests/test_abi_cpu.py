"""C ABI checks that need no GPU: the library loads, exports every function
include/nest_splat.h declares, reports layouts, and rejects bad arguments
before launching anything (error codes and messages, outputs untouched)."""
import ctypes as ct
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    from nest_splat import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.fail(f"{L.LIB_PATH} not built (run __graft_entry__.build())")
    return L


def declared_functions():
    src = open(os.path.join(ROOT, "include", "nest_splat.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char \*)\s*(nest_\w+)\(", src, re.M)))


def test_exports_match_header():
    L = _lib()
    lib = L.lib()
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
        assert n in L.EXPORTS, f"{n} has no ctypes signature"
    src = open(os.path.join(ROOT, "include", "nest_splat.h")).read()
    header_version = int(re.search(r"#define NEST_ABI_VERSION (\d+)", src).group(1))
    assert lib.nest_abi_version() == header_version == L.ABI_VERSION
    # render-mode constants: the header's values are the Python side's
    modes = dict(re.findall(r"#define NEST_(MODE_\w+) (0x[0-9A-Fa-f]+|\d+)", src))
    assert len(modes) >= 7
    for name, value in modes.items():
        assert getattr(L, name) == int(value, 0), name


def test_struct_sizes_match_c_layout():
    """ctypes mirrors of the ABI structs have the sizes the library checks
    (a mismatch is reported as NEST_ERR_INVALID_ARGUMENT, see below)."""
    L = _lib()
    assert ct.sizeof(L.RasterSettings) == 4 * (6 + 16 + 16 + 3 + 1 + 4)
    assert ct.sizeof(L.HashGrid) % 8 == 0
    assert ct.sizeof(L.Splats) == 8 + 9 * 8 + 16
    assert ct.sizeof(L.FrameOutputs) == 8 + 5 * 8
    assert ct.sizeof(L.Mlp) == 16 + 3 * 8
    assert ct.sizeof(L.BackwardIO) == 8 + 12 * 8


def test_layouts_are_aligned_and_monotone():
    L = _lib()
    for P in (0, 1, 1000, 1 << 20):
        offs, tot = L.geom_layout(P)
        assert all(o % 256 == 0 for o in offs) and offs == sorted(offs) and tot >= offs[-1]
        assert offs[L.GEOM_RECORDS + 1] - offs[L.GEOM_RECORDS] >= max(P, 1) * 128
        assert offs[L.GEOM_ORDER_TMP] - offs[L.GEOM_DEPTH_ORDER] >= max(P, 1) * 8
        assert tot - offs[L.GEOM_ORDER_TMP] >= max(P, 1) * 16  # depth keys + sort ping-pong
    offs, tot = L.binning_layout(5_000_000)
    assert offs[L.BIN_KEYS] - offs[L.BIN_PAIR_TILES] >= 5_000_000 * 8
    assert offs[L.BIN_SORT_TMP] - offs[L.BIN_KEYS] >= 5_000_000 * 12
    assert tot - offs[L.BIN_SORT_TMP] >= 5_000_000 * 16  # two u32 key/value ping-pong sets
    offs, tot = L.image_layout(1600, 1064)
    assert offs[L.IMG_FINAL_T] >= 6700 * 8 and tot >= 1600 * 1064 * 20


def _settings(L, **kw):
    s = L.RasterSettings()
    s.struct_size = ct.sizeof(L.RasterSettings)
    s.image_height, s.image_width = 64, 64
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def _splats(L, P=10):
    sp = L.Splats()
    sp.struct_size = ct.sizeof(L.Splats)
    sp.P = P
    return sp


def test_geometry_rejects_bad_arguments():
    L = _lib()
    lib = L.lib()
    nr = ct.c_int64(-7)
    tm = L.Timing()
    ws = (ct.c_uint8 * 16)()
    # wrong struct size
    s = _settings(L, struct_size=3)
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(_splats(L)), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_INVALID_ARGUMENT and b"struct_size" in lib.nest_last_error()
    # non-positive image
    s = _settings(L, image_width=0)
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(_splats(L)), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_INVALID_ARGUMENT and b"image size" in lib.nest_last_error()
    # missing attribute pointers
    s = _settings(L)
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(_splats(L)), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_INVALID_ARGUMENT and b"required" in lib.nest_last_error()
    # workspace too small (pointers are never dereferenced on this path)
    sp = _splats(L)
    sp.means3D = sp.scales = sp.rotations = sp.opacities = 1
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(sp), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_WORKSPACE and b"too small" in lib.nest_last_error()
    assert nr.value == -7  # outputs untouched on error
    # prefiltered is unsupported
    s = _settings(L, prefiltered=1)
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(sp), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_UNSUPPORTED
    # SH colours: degree 0..3 with enough coefficients per splat
    s = _settings(L)
    sp.shs, sp.sh_degree, sp.sh_coeffs = 1, 4, 25
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(sp), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_UNSUPPORTED and b"degree" in lib.nest_last_error()
    sp.sh_degree, sp.sh_coeffs = 3, 9
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(sp), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_INVALID_ARGUMENT and b"coefficients" in lib.nest_last_error()
    # with precomputed colours the SH arguments are not used
    sp.colors_precomp = 1
    rc = lib.nest_forward_geometry(ct.byref(s), ct.byref(sp), ws, 16, None, ct.byref(nr), ct.byref(tm), None)
    assert rc == L.NEST_ERR_WORKSPACE


def test_render_rejects_bad_grids():
    L = _lib()
    lib = L.lib()
    s = _settings(L)
    sp = _splats(L, 0)
    g = L.HashGrid()
    g.struct_size = ct.sizeof(L.HashGrid)
    g.levels, g.level_dim = 16, 3
    out = L.FrameOutputs()
    out.struct_size = ct.sizeof(L.FrameOutputs)
    out.channels = 48
    out.out_color = out.out_others = 1
    ws = (ct.c_uint8 * 16)()
    args = lambda: (ct.byref(s), ct.byref(g), ct.byref(sp), ws, 16, ws, 16, ws, 16, 0, ct.byref(out), None, None)
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED  # level_dim 3
    g.level_dim = 4
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # 48 < 64 channels
    assert b"channels" in lib.nest_last_error()
    out.channels = 64
    g.table = 1
    g.table_rows = 10
    g.gridrange[0], g.gridrange[1] = -1.0, 1.0
    for i in range(17):
        g.offsets[i] = i * 1024
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # table too small
    assert b"rows" in lib.nest_last_error()
    g.table_rows = 16 * 1024
    g.offsets[5] = g.offsets[4]
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # empty level
    g.offsets[5] = 5 * 1024
    g.gridrange[1] = -1.0
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # empty range
    g.gridrange[1] = 1.0
    out.channels = 200
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED
    out.channels = 64
    # workspace checks come after argument checks and before any launch
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_WORKSPACE


def test_render_validates_hybrid_sh_modes():
    """Render modes 8-10: one float32 grid level of 3 channels, rows in
    colors_precomp, 3 or 48 output channels, decompose 0-2; checked before
    any launch."""
    L = _lib()
    lib = L.lib()
    s = _settings(L)
    sp = _splats(L, 0)
    g = L.HashGrid()
    g.struct_size = ct.sizeof(L.HashGrid)
    g.render_mode = L.MODE_HYBRID_SH_POST
    g.levels, g.level_dim, g.table, g.table_rows = 1, 3, 1, 4096
    g.offsets[1] = 4096
    g.gridrange[0], g.gridrange[1] = -1.0, 1.0
    out = L.FrameOutputs()
    out.struct_size = ct.sizeof(L.FrameOutputs)
    out.channels = 3
    out.out_color = out.out_others = 1
    ws = (ct.c_uint8 * 16)()
    args = lambda: (ct.byref(s), ct.byref(g), ct.byref(sp), ws, 16, ws, 16, ws, 16, 0, ct.byref(out), None, None)
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # mode 9 writes 48 channels
    assert b"48" in lib.nest_last_error()
    out.channels = 48
    g.levels = 2
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED  # one level
    g.levels, g.level_dim = 1, 4
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED  # level_dim 3
    g.level_dim, g.table_dtype = 3, L.DTYPE_F16
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED  # float32 table
    g.table_dtype, g.decompose = L.DTYPE_F32, 3
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT
    g.decompose = 2
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_WORKSPACE  # arguments accepted
    g.render_mode, out.channels = L.MODE_HYBRID_SH, 3
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_WORKSPACE


def test_render_validates_dual_grid_modes():
    """Render modes 2 and 3: level_dim 4, at most 64 channels, a valid second
    grid when given, the rows2 scratch; checked before any launch."""
    L = _lib()
    lib = L.lib()
    s = _settings(L)
    sp = _splats(L, 0)
    g = L.HashGrid()
    g.struct_size = ct.sizeof(L.HashGrid)
    g.render_mode = L.MODE_BASELINE_DOUBLE
    g.levels, g.level_dim, g.table, g.table_rows = 8, 4, 1, 8 * 1024
    for i in range(9):
        g.offsets[i] = g.offsets2[i] = i * 1024
    g.gridrange[0], g.gridrange[1] = -1.0, 1.0
    out = L.FrameOutputs()
    out.struct_size = ct.sizeof(L.FrameOutputs)
    out.channels = 32
    out.out_color = out.out_others = 1
    ws = (ct.c_uint8 * 16)()
    args = lambda: (ct.byref(s), ct.byref(g), ct.byref(sp), ws, 16, ws, 16, ws, 16, 0, ct.byref(out), None, None)
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # mode 2 writes 64 channels
    out.channels = 64
    g.levels = 9
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED  # 72 channels
    g.levels, g.level_dim = 8, 2
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_UNSUPPORTED  # level_dim 4
    g.level_dim, g.table2, g.table2_rows = 4, 1, 10
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # second table too small
    g.table2_rows = 8 * 1024
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # empty gridrange2
    g.gridrange2[0], g.gridrange2[1] = -2.0, 2.0
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_WORKSPACE  # accepted
    g.render_mode, g.levels = L.MODE_BASELINE_BLEND_DOUBLE, 16
    for i in range(17):
        g.offsets[i] = g.offsets2[i] = i * 512
    assert lib.nest_forward_render(*args()) == L.NEST_ERR_WORKSPACE  # mode 3: 16 levels, 64 channels


def test_backward_layout_and_validation():
    """nest_backward_layout sizes and the argument checks of nest_backward /
    nest_grid_encode_backward, which return before any launch."""
    L = _lib()
    lib = L.lib()
    offs = (ct.c_size_t * L.BWD_FIELDS)()
    tot = ct.c_size_t(0)
    assert lib.nest_backward_layout(1000, 64, offs, ct.byref(tot)) == L.NEST_OK
    o = list(offs)
    assert all(v % 256 == 0 for v in o) and o == sorted(o)
    assert o[L.BWD_DHOMO] - o[L.BWD_DTRANSMAT] >= 1000 * 36 and o[L.BWD_GRADSUM] - o[L.BWD_DCOLORS] >= 1000 * 256
    assert tot.value >= o[L.BWD_GRADSUM] + 4000
    assert lib.nest_backward_layout(-1, 3, offs, ct.byref(tot)) == L.NEST_ERR_INVALID_ARGUMENT
    s = _settings(L)
    sp = _splats(L, 0)
    g = L.HashGrid()
    g.struct_size = ct.sizeof(L.HashGrid)
    io = L.BackwardIO()
    io.struct_size = ct.sizeof(L.BackwardIO)
    io.channels = 3
    ws = (ct.c_uint8 * 16)()
    args = lambda: (ct.byref(s), ct.byref(g), ct.byref(sp), ws, 16, ws, 16, ws, 16, 0, ct.byref(io), ws, 16, None)
    assert lib.nest_backward(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # no gradient inputs
    assert b"dL_dout_color" in lib.nest_last_error()
    io.dL_dout_color = io.dL_dout_others = 1
    assert lib.nest_backward(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # no outputs
    io.dL_dmeans3D = io.dL_dmeans2D = io.dL_dopacity = io.dL_dscales = io.dL_drotations = 1
    io.channels = 65
    assert lib.nest_backward(*args()) == L.NEST_ERR_UNSUPPORTED  # more than 64 channels
    io.channels = 64
    g.levels, g.level_dim, g.table, g.table_rows = 16, 4, 1, 16 * 1024
    g.table_dtype = L.DTYPE_F16
    g.gridrange[0], g.gridrange[1] = -1.0, 1.0
    for i in range(17):
        g.offsets[i] = i * 1024
    assert lib.nest_backward(*args()) == L.NEST_ERR_UNSUPPORTED  # binary16 table
    assert b"float32" in lib.nest_last_error()
    g.table_dtype = L.DTYPE_F32
    assert lib.nest_backward(*args()) == L.NEST_ERR_INVALID_ARGUMENT  # no dL_dfeatures
    io.dL_dfeatures = 1
    assert lib.nest_backward(*args()) == L.NEST_ERR_WORKSPACE
    io.struct_size = 8
    assert lib.nest_backward(*args()) == L.NEST_ERR_INVALID_ARGUMENT
    offs32 = (ct.c_int32 * 3)(0, 64, 128)
    ge = lambda D, dt: lib.nest_grid_encode_backward(1, 4, D, 1, 128, dt, offs32, 2, 2, 0.5, 4, 0, 0, 0, 1, 1, None,
                                                      None)
    assert ge(2, L.DTYPE_F32) == L.NEST_ERR_UNSUPPORTED
    assert ge(3, L.DTYPE_F16) == L.NEST_ERR_UNSUPPORTED


def test_building_block_validation():
    L = _lib()
    lib = L.lib()
    assert lib.nest_sort_workspace_size(1000) > 1000 * 12
    assert lib.nest_scan_workspace_size(1 << 20) >= 8 * 256
    assert lib.nest_sort_pairs_u64(None, None, None, None, 10, 70, None, 0, None) == L.NEST_ERR_INVALID_ARGUMENT
    assert lib.nest_sort_pairs_u64(None, None, None, None, 0, 45, None, 0, None) == L.NEST_OK
    assert lib.nest_inclusive_scan_u32(None, None, -1, None, 0, None) == L.NEST_ERR_INVALID_ARGUMENT
    view = (ct.c_float * 16)()
    assert lib.nest_mark_visible(-1, None, view, None, None) == L.NEST_ERR_INVALID_ARGUMENT
    assert lib.nest_mark_visible(0, None, view, None, None) == L.NEST_OK
    assert lib.nest_mark_visible(5, None, view, None, None) == L.NEST_ERR_INVALID_ARGUMENT
    offs = (ct.c_int32 * 17)(*[i * 64 for i in range(17)])
    assert lib.nest_grid_encode(None, 10, 6, None, 0, 0, offs, 16, 2, 0.5, 16, 0, 0, 0, None, None) == L.NEST_ERR_UNSUPPORTED
    assert lib.nest_grid_encode(None, 10, 3, None, 0, 0, offs, 16, 3, 0.5, 16, 0, 0, 0, None, None) == L.NEST_ERR_UNSUPPORTED
    assert lib.nest_grid_encode(None, 10, 3, None, 100, 0, offs, 16, 2, 0.5, 16, 0, 0, 0, None, None) == \
        L.NEST_ERR_INVALID_ARGUMENT  # 100 rows < offsets[16]
    m = L.Mlp()
    m.struct_size = ct.sizeof(L.Mlp)
    m.in_features, m.width, m.dtype = 24, 64, L.DTYPE_BF16
    assert lib.nest_mlp_decode(ct.byref(m), None, 1, 1, 10, 8, None, None, None, None, None, 1, 1, None) == \
        L.NEST_ERR_UNSUPPORTED  # MFMA path needs C % 16 == 0
    m.in_features, m.width = 32, 48
    assert lib.nest_mlp_decode(ct.byref(m), None, 1, 1, 10, 8, None, None, None, None, None, 1, 1, None) == \
        L.NEST_ERR_UNSUPPORTED
    assert lib.nest_rvq_decode(10, 4, 4096, 5, None, None, None, 0, None, None, None) == L.NEST_ERR_UNSUPPORTED
    assert lib.nest_rvq_decode(10, 4, 4096, 2, None, None, None, 7, None, None, None) == L.NEST_ERR_INVALID_ARGUMENT
    attrs = (L.RvqAttr * 5)()
    for a in attrs:
        a.struct_size, a.P, a.stages, a.codebook_size, a.dim = ct.sizeof(L.RvqAttr), 0, 4, 4096, 2
    assert lib.nest_rvq_decode_batch(5, attrs, None) == L.NEST_ERR_INVALID_ARGUMENT  # at most 4 attributes
    assert lib.nest_rvq_decode_batch(3, attrs, None) == L.NEST_OK  # empty attributes launch nothing
    attrs[1].dim = 5
    assert lib.nest_rvq_decode_batch(3, attrs, None) == L.NEST_ERR_UNSUPPORTED
    attrs[1].dim, attrs[2].struct_size = 2, 8
    assert lib.nest_rvq_decode_batch(3, attrs, None) == L.NEST_ERR_INVALID_ARGUMENT


def test_python_errors_are_raised():
    L = _lib()
    with pytest.raises(NotImplementedError):
        L.check(L.NEST_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        L.check(L.NEST_ERR_HIP, "x")
