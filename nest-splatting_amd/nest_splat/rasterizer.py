"""Forward rasterisation through libnest_splat: the host side of
RasterizeGaussiansCUDA (submodules/diff-surfel-rasterization/
rasterize_points.cu:40-242) for render mode 0.

Outputs and workspaces are torch tensors on the splats' device; the library
fills them with stream-ordered kernels on torch's current stream.  The one
host synchronisation is the tile/splat pair count read back between the
geometry and render stages, exactly where the reference reads num_rendered.
"""
from __future__ import annotations

import dataclasses

import ctypes as ct
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np
import torch

from . import _lib as L


def host_array(x, dtype) -> np.ndarray:
    """Host copy of a small tensor or array.  Device tensors are copied once
    (a synchronisation) and the copy is cached on the tensor object."""
    if isinstance(x, torch.Tensor):
        cached = getattr(x, "_nest_host_copy", None)
        if cached is not None and cached[0] == x._version:
            return cached[1]
        arr = x.detach().cpu().numpy().astype(dtype).reshape(-1)
        try:
            x._nest_host_copy = (x._version, arr)
        except Exception:
            pass
        return arr
    return np.asarray(x, dtype=dtype).reshape(-1)


@dataclass
class HashGridDesc:
    """Hash grid seen by the render kernel (HashGridSettings + get_params)."""

    levels: int
    level_dim: int
    log2_scale: float
    base_resolution: int
    table: Optional[torch.Tensor]
    offsets: np.ndarray
    gridrange: np.ndarray
    align_corners: bool = False
    interpolation: int = 0
    # render_mode 4 / 7 / 12 / 13 / 14 (| MODE_INFERENCE): per-splat feature levels ahead
    # of the grid's `levels` (hybrid_levels) and, for modes 12/13, the levels of a
    # splat's feature row (total_levels; the row ends with the blend weight)
    render_mode: int = 0
    hybrid_levels: int = 0
    total_levels: int = 0
    # render_mode 4 backward: the grid levels it differentiates are those up to
    # the active count (coarse-to-fine training); None = all `levels`
    active_levels: Optional[int] = None
    # render_mode 8 / 9 / 10 (hybrid SH): 0 both parts, 1 gaussian_only, 2 ngp_only
    decompose: int = 0
    # render_mode 1 / 2 / 3: the second grid (float32 [rows, 4] table, offsets, range)
    # queried at the splat centres; table2 None leaves its features 0
    table2: Optional[torch.Tensor] = None
    offsets2: Optional[np.ndarray] = None
    gridrange2: Optional[np.ndarray] = None
    rows2: Optional[torch.Tensor] = None  # [P, levels * 4] scratch, set by rasterize_forward

    def dual(self) -> bool:
        """Render modes 1, 2, 3 and 5: features at the splat centres, in rows2."""
        return (self.render_mode & 0xFF) in (L.MODE_SURFACE, L.MODE_BASELINE_DOUBLE, L.MODE_BASELINE_BLEND_DOUBLE,
                                             L.MODE_SURFACE_RGB)

    def row_width(self, channels: int) -> int:
        """Floats per splat of colors_precomp for this render mode."""
        base = self.render_mode & 0xFF
        if base in (L.MODE_HYBRID_SH, L.MODE_HYBRID_SH_RAW):
            return 3
        if base == L.MODE_HYBRID_SH_POST:
            return 48
        if base == L.MODE_CAT:
            return self.hybrid_levels * self.level_dim
        if base == L.MODE_ADAPTIVE_ZERO:
            return self.hybrid_levels * self.level_dim + 1
        if base in (L.MODE_ADAPTIVE_ADD, L.MODE_ADAPTIVE_CAT, L.MODE_ADAPTIVE_CAT_FAST):
            return self.total_levels * self.level_dim + 1
        return channels

    def to_c(self) -> L.HashGrid:
        g = L.HashGrid()
        g.struct_size = ct.sizeof(L.HashGrid)
        g.render_mode = int(self.render_mode)
        g.hybrid_levels = int(self.hybrid_levels)
        g.total_levels = int(self.total_levels)
        g.active_levels = int(self.levels if self.active_levels is None else self.active_levels)
        g.decompose = int(self.decompose)
        g.levels = int(self.levels)
        g.level_dim = int(self.level_dim)
        g.log2_scale = float(self.log2_scale)
        g.base_resolution = int(self.base_resolution)
        g.align_corners = int(bool(self.align_corners))
        g.interpolation = int(self.interpolation)
        if self.levels > 0:
            t = self.table
            if t.dtype == torch.float32:
                g.table_dtype = L.DTYPE_F32
            elif t.dtype == torch.float16:
                g.table_dtype = L.DTYPE_F16
            else:
                raise NotImplementedError(f"hash table dtype {t.dtype} is not supported (float32/float16)")
            if not t.is_contiguous():
                raise ValueError("hash table must be contiguous")
            if not t.is_cuda:
                raise ValueError("hash table must be a device tensor")
            if t.data_ptr() % 16 != 0:
                t = self.table = t.clone()
            g.table = t.data_ptr()
            g.table_rows = int(t.shape[0])
            if self.levels > L.MAX_LEVELS:
                raise NotImplementedError(f"at most {L.MAX_LEVELS} levels")
            offs = np.asarray(self.offsets, dtype=np.int64)
            if offs.shape[0] < self.levels + 1:
                raise ValueError(f"offsets has {offs.shape[0]} entries, need {self.levels + 1}")
            for i in range(self.levels + 1):
                g.offsets[i] = int(offs[i])
            g.gridrange[0] = float(self.gridrange[0])
            g.gridrange[1] = float(self.gridrange[1])
        if self.dual():
            if self.table2 is not None:
                t2 = self.table2
                if t2.dtype != torch.float32 or not t2.is_cuda or t2.dim() != 2 or t2.shape[1] != 4:
                    raise ValueError("the second grid's table must be a float32 [rows, 4] device tensor")
                if not t2.is_contiguous() or t2.data_ptr() % 16 != 0:
                    t2 = self.table2 = t2.contiguous().clone()
                g.table2 = t2.data_ptr()
                g.table2_rows = int(t2.shape[0])
                o2 = np.asarray(self.offsets2, dtype=np.int64)
                if o2.shape[0] < self.levels + 1:
                    raise ValueError(f"offsets2 has {o2.shape[0]} entries, need {self.levels + 1}")
                for i in range(self.levels + 1):
                    g.offsets2[i] = int(o2[i])
                g.gridrange2[0] = float(self.gridrange2[0])
                g.gridrange2[1] = float(self.gridrange2[1])
            g.rows2 = L.ptr(self.rows2).value if self.rows2 is not None else None
        return g


def make_settings(H: int, W: int, tanfovx: float, tanfovy: float, viewmatrix, projmatrix, campos=(0, 0, 0),
                  scale_modifier: float = 1.0, beta: float = 0.0, if_contract: bool = False,
                  max_intersections: int = 0, prefiltered: bool = False, debug: bool = False) -> L.RasterSettings:
    s = L.RasterSettings()
    s.struct_size = ct.sizeof(L.RasterSettings)
    s.image_height = int(H)
    s.image_width = int(W)
    s.tanfovx = float(tanfovx)
    s.tanfovy = float(tanfovy)
    s.scale_modifier = float(scale_modifier)
    vm = host_array(viewmatrix, np.float32)
    pm = host_array(projmatrix, np.float32)
    cp = host_array(campos, np.float32)
    for i in range(16):
        s.viewmatrix[i] = float(vm[i])
        s.projmatrix[i] = float(pm[i])
    for i in range(3):
        s.campos[i] = float(cp[i]) if cp.size == 3 else 0.0
    s.beta = float(beta)
    s.prefiltered = int(bool(prefiltered))
    s.debug = int(bool(debug))
    s.if_contract = int(bool(if_contract))
    s.max_intersections = int(max_intersections)
    return s


@dataclass
class ForwardResult:
    num_rendered: int
    color: torch.Tensor
    others: torch.Tensor
    radii: torch.Tensor
    geom: torch.Tensor
    binning: torch.Tensor
    image: torch.Tensor
    timing_ms: Dict[str, float] = field(default_factory=dict)
    # record_transmittance: hits per splat and the sum of the transmittance
    # before each of them, [P] each (None when not recorded)
    cover_pixels: Optional[torch.Tensor] = None
    trans_avg: Optional[torch.Tensor] = None


def aligned(t: torch.Tensor, align: int = 16) -> torch.Tensor:
    """Contiguous tensor whose data pointer is a multiple of ``align`` bytes
    (the kernels read splat attributes and table rows with 8/16-byte loads)."""
    t = t.contiguous()
    if t.data_ptr() % align != 0:
        t = t.clone()
    return t


def _contig_f32(t: Optional[torch.Tensor], name: str) -> Optional[torch.Tensor]:
    if t is None or t.numel() == 0:
        return None
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (got {t.dtype})")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    return aligned(t)


def _splats(means3D, opacities, scales, rotations, homotrans, ap_level, colors_precomp, channels, shs, sh_degree,
            row_width=None, shapes=None, kernel_type=0):
    """nest_splats over the device tensors (re-aligned copies where needed);
    returns (struct, tensors kept alive for the call)."""
    if means3D.ndim != 2 or means3D.shape[1] != 3:
        raise ValueError("means3D must have dimensions (num_points, 3)")
    P = int(means3D.shape[0])
    means3D = _contig_f32(means3D, "means3D")
    opacities = _contig_f32(opacities, "opacities")
    scales = _contig_f32(scales, "scales")
    rotations = _contig_f32(rotations, "rotations")
    homotrans = _contig_f32(homotrans, "homotrans")
    ap_level = _contig_f32(ap_level, "ap_level")
    colors_precomp = _contig_f32(colors_precomp, "colors_precomp")
    shs = _contig_f32(shs, "shs") if shs is not None and shs.numel() > 0 else None
    shapes = _contig_f32(shapes, "shapes") if kernel_type != 0 else None
    if P > 0:
        if kernel_type != 0 and (shapes is None or shapes.numel() != P):
            raise ValueError(f"kernel_type {kernel_type} needs shapes with P elements")
        for t, n, k in ((scales, "scales", 2), (rotations, "rotations", 4)):
            if t is None or t.numel() != P * k:
                raise ValueError(f"{n} must have {P}x{k} elements")
        if opacities is None or opacities.numel() != P:
            raise ValueError("opacities must have P elements")
        if homotrans is not None and homotrans.numel() != P * 16:
            raise ValueError("homotrans must be [P, 4, 4]")
        if ap_level is not None and ap_level.numel() != P:
            raise ValueError("ap_level must have P elements")
        width = channels if row_width is None else row_width
        if colors_precomp is not None and colors_precomp.numel() != P * width:
            raise ValueError(f"colors_precomp must be [P, {width}]")
        if shs is not None and (shs.numel() % (P * 3) != 0 or shs.shape[0] != P):
            raise ValueError("shs must be [P, M, 3]")

    sp = L.Splats()
    sp.struct_size = ct.sizeof(L.Splats)
    sp.P = P
    sp.means3D = L.ptr(means3D)
    sp.scales = L.ptr(scales)
    sp.rotations = L.ptr(rotations)
    sp.opacities = L.ptr(opacities)
    sp.homotrans = L.ptr(homotrans)
    sp.ap_level = L.ptr(ap_level)
    sp.colors_precomp = L.ptr(colors_precomp)
    sp.shs = L.ptr(shs)
    sp.sh_degree = int(sh_degree)
    sp.sh_coeffs = int(shs.numel() // (3 * P)) if shs is not None and P > 0 else 0
    sp.shapes = L.ptr(shapes)
    sp.kernel_type = int(kernel_type)
    return sp, (means3D, opacities, scales, rotations, homotrans, ap_level, colors_precomp, shs, shapes)


def rasterize_forward(settings: L.RasterSettings, grid: HashGridDesc, means3D: torch.Tensor, opacities: torch.Tensor,
                      scales: torch.Tensor, rotations: torch.Tensor, homotrans: Optional[torch.Tensor] = None,
                      ap_level: Optional[torch.Tensor] = None, colors_precomp: Optional[torch.Tensor] = None,
                      channels: int = 3, timing: bool = False, shs: Optional[torch.Tensor] = None,
                      sh_degree: int = 0, record_transmittance: bool = False, shapes: Optional[torch.Tensor] = None,
                      kernel_type: int = 0) -> ForwardResult:
    """One forward frame.  The colour path (grid.levels == 0 in render mode
    0) takes colours from colors_precomp, or, when it is None, evaluates them
    from shs [P, M, 3] at degree sh_degree in preprocess (3 channels).  In
    render modes 4 and 13 colors_precomp holds the per-splat feature rows
    (grid.row_width floats each).  record_transmittance fills
    cover_pixels / trans_avg (DSR/rasterize_points.cu:169-171,
    CR/forward.cu:1961-1964).  kernel_type 1 (beta), 2 (flex) or 3 (general)
    takes the per-splat parameter from shapes [P] (CR/forward.cu:864-900)."""
    dev = means3D.device
    P = int(means3D.shape[0])
    H, W = settings.image_height, settings.image_width
    sp, keep = _splats(means3D, opacities, scales, rotations, homotrans, ap_level, colors_precomp, channels, shs,
                       sh_degree, grid.row_width(channels), shapes=shapes, kernel_type=kernel_type)
    if grid.dual():
        # render modes 2 and 3: scratch for the second grid's features at the splat centres
        grid = dataclasses.replace(grid, rows2=torch.empty((max(P, 1), grid.levels * 4), dtype=torch.float32,
                                                           device=dev))
    g = grid.to_c()

    color = torch.empty((channels, H, W), dtype=torch.float32, device=dev)
    others = torch.empty((L.OTHERS_CHANNELS, H, W), dtype=torch.float32, device=dev)
    radii = torch.zeros((P,), dtype=torch.int32, device=dev)
    _, gbytes = L.geom_layout(P)
    geom = torch.empty((gbytes,), dtype=torch.uint8, device=dev)
    _, ibytes = L.image_layout(W, H)
    image = torch.empty((ibytes,), dtype=torch.uint8, device=dev)
    own_timing = not isinstance(timing, L.Timing)
    tm = L.new_timing(bool(timing)) if own_timing else timing
    stream = L.stream_ptr(dev)
    nr = ct.c_int64(0)
    lib = L.lib()
    L.check(lib.nest_forward_geometry(ct.byref(settings), ct.byref(sp), L.ptr(geom), gbytes, L.ptr(radii),
                                      ct.byref(nr), ct.byref(tm), stream), "nest_forward_geometry")
    NR = int(nr.value)
    _, bbytes = L.binning_layout(NR)
    binning = torch.empty((bbytes,), dtype=torch.uint8, device=dev)
    out = L.FrameOutputs()
    out.struct_size = ct.sizeof(L.FrameOutputs)
    out.channels = int(channels)
    out.out_color = color.data_ptr()
    out.out_others = others.data_ptr()
    out.radii = radii.data_ptr()
    cover = trans = None
    if record_transmittance:
        cover = torch.empty((P,), dtype=torch.float32, device=dev)
        trans = torch.empty((P,), dtype=torch.float32, device=dev)
        out.cover_pixels = cover.data_ptr() if P > 0 else None
        out.trans_avg = trans.data_ptr() if P > 0 else None
    L.check(lib.nest_forward_render(ct.byref(settings), ct.byref(g), ct.byref(sp), L.ptr(geom), gbytes,
                                    L.ptr(binning), bbytes, L.ptr(image), ibytes, NR, ct.byref(out), ct.byref(tm),
                                    stream), "nest_forward_render")
    res = ForwardResult(NR, color, others, radii, geom, binning, image, cover_pixels=cover, trans_avg=trans)
    if own_timing and timing:
        res.timing_ms = L.timing_read(tm)
        L.timing_release(tm)
    return res


@dataclass
class BackwardResult:
    dmeans3D: torch.Tensor      # [P, 3]
    dmeans2D: torch.Tensor      # [P, 3] densification statistic of the reference
    dcolors: torch.Tensor       # [P, C]
    dopacity: torch.Tensor      # [P, 1]
    dshs: Optional[torch.Tensor]  # [P, M, 3] when the colours came from SH
    dscales: torch.Tensor       # [P, 2]
    drotations: torch.Tensor    # [P, 4]
    dfeatures: Optional[torch.Tensor]  # [rows, F] hash path
    dgradsum: torch.Tensor      # [P, 1]
    dshapes: Optional[torch.Tensor] = None  # [P] kernel types 1-3


def rasterize_backward(settings: L.RasterSettings, grid: HashGridDesc, res: ForwardResult, means3D: torch.Tensor,
                       opacities: torch.Tensor, scales: torch.Tensor, rotations: torch.Tensor,
                       dL_dcolor: torch.Tensor, dL_dothers: Optional[torch.Tensor],
                       homotrans: Optional[torch.Tensor] = None, ap_level: Optional[torch.Tensor] = None,
                       colors_precomp: Optional[torch.Tensor] = None, channels: int = 3,
                       shs: Optional[torch.Tensor] = None, sh_degree: int = 0, shapes: Optional[torch.Tensor] = None,
                       kernel_type: int = 0) -> BackwardResult:
    """Backward of one forward frame (nest_backward): the inputs are those
    of the rasterize_forward call that produced ``res``."""
    dev = means3D.device
    P = int(means3D.shape[0])
    H, W = settings.image_height, settings.image_width
    sp, keep = _splats(means3D, opacities, scales, rotations, homotrans, ap_level, colors_precomp, channels, shs,
                       sh_degree, grid.row_width(channels), shapes=shapes, kernel_type=kernel_type)
    g = grid.to_c()
    if dL_dcolor is None:
        dL_dcolor = torch.zeros((channels, H, W), dtype=torch.float32, device=dev)
    if dL_dothers is None:
        dL_dothers = torch.zeros((L.OTHERS_CHANNELS, H, W), dtype=torch.float32, device=dev)
    dL_dcolor = dL_dcolor.to(torch.float32).contiguous()
    dL_dothers = dL_dothers.to(torch.float32).contiguous()
    if tuple(dL_dcolor.shape) != (channels, H, W) or tuple(dL_dothers.shape) != (L.OTHERS_CHANNELS, H, W):
        raise ValueError("gradient shapes must match the forward outputs")
    f32 = dict(dtype=torch.float32, device=dev)
    out = BackwardResult(
        dmeans3D=torch.empty((P, 3), **f32), dmeans2D=torch.empty((P, 3), **f32),
        dcolors=torch.empty((P, grid.row_width(channels)), **f32), dopacity=torch.empty((P, 1), **f32),
        dshs=None, dscales=torch.empty((P, 2), **f32), drotations=torch.empty((P, 4), **f32),
        dfeatures=None, dgradsum=torch.empty((P, 1), **f32))
    if kernel_type != 0:
        out.dshapes = torch.empty((P,), **f32)
    if grid.levels > 0:
        out.dfeatures = torch.empty(tuple(grid.table.shape), **f32)
    elif colors_precomp is None or colors_precomp.numel() == 0:
        out.dshs = torch.empty(tuple(shs.shape), **f32)
    io = L.BackwardIO()
    io.struct_size = ct.sizeof(L.BackwardIO)
    io.channels = int(channels)
    io.dL_dout_color = dL_dcolor.data_ptr()
    io.dL_dout_others = dL_dothers.data_ptr()
    io.dL_dmeans3D = out.dmeans3D.data_ptr()
    io.dL_dmeans2D = out.dmeans2D.data_ptr()
    io.dL_dcolors = out.dcolors.data_ptr()
    io.dL_dopacity = out.dopacity.data_ptr()
    io.dL_dshs = L.ptr(out.dshs)
    io.dL_dscales = out.dscales.data_ptr()
    io.dL_drotations = out.drotations.data_ptr()
    io.dL_dfeatures = L.ptr(out.dfeatures)
    io.dL_dgradsum = out.dgradsum.data_ptr()
    io.dL_dshapes = L.ptr(out.dshapes)
    offs = (ct.c_size_t * L.BWD_FIELDS)()
    wbytes = ct.c_size_t(0)
    L.check(L.lib().nest_backward_layout(P, int(channels), offs, ct.byref(wbytes)), "nest_backward_layout")
    ws = torch.empty((max(int(wbytes.value), 1),), dtype=torch.uint8, device=dev)
    L.check(L.lib().nest_backward(ct.byref(settings), ct.byref(g), ct.byref(sp), L.ptr(res.geom), res.geom.numel(),
                                  L.ptr(res.binning), res.binning.numel(), L.ptr(res.image), res.image.numel(),
                                  res.num_rendered, ct.byref(io), L.ptr(ws), int(wbytes.value), L.stream_ptr(dev)),
            "nest_backward")
    return out


def geometry_arrays(res: ForwardResult, P: int) -> Dict[str, torch.Tensor]:
    """Typed views of the geometry workspace (for tests and debugging)."""
    o, _ = L.geom_layout(P)
    n = max(P, 1)
    return dict(depth=L.view(res.geom, o[L.GEOM_DEPTH], torch.float32, (n,))[:P],
                xy=L.view(res.geom, o[L.GEOM_XY], torch.float32, (n, 2))[:P],
                tiles=L.view(res.geom, o[L.GEOM_TILES], torch.int32, (n,))[:P],
                offsets=L.view(res.geom, o[L.GEOM_OFFSETS], torch.int32, (n,))[:P],
                records=L.view(res.geom, o[L.GEOM_RECORDS], torch.float32, (n, 32))[:P],
                radii=L.view(res.geom, o[L.GEOM_RADII], torch.int32, (n,))[:P],
                depth_order=L.view(res.geom, o[L.GEOM_DEPTH_ORDER], torch.int32, (n,))[:P],
                order_offsets=L.view(res.geom, o[L.GEOM_ORDER_OFFSETS], torch.int32, (n,))[:P],
                rgb=L.view(res.geom, o[L.GEOM_RGB], torch.float32, (n, 3))[:P],
                clamped=L.view(res.geom, o[L.GEOM_CLAMPED], torch.uint8, (n, 3))[:P])


def build_homotrans(rotations: torch.Tensor, scales: torch.Tensor, means3D: torch.Tensor) -> torch.Tensor:
    """get_homotrans (scene/gaussian_model.py:312-317): build_H(build_rotation
    (rotations), scales, means3D) of utils/general_utils.py:78-113 on the GPU,
    [P, 4, 4] float32, bit-exact with the reference's torch expressions.
    rotations are the raw quaternions (GaussianModel._rotation): build_rotation
    normalises them, as the kernel does."""
    P = int(rotations.shape[0])
    if rotations.shape != (P, 4) or scales.shape != (P, 2) or means3D.shape != (P, 3):
        raise ValueError("rotations [P,4], scales [P,2] and means3D [P,3] are required")
    out = torch.empty((P, 4, 4), dtype=torch.float32, device=rotations.device)
    if P == 0:
        return out
    rot = _contig_f32(rotations, "rotations")
    sc = _contig_f32(scales, "scales")
    mn = _contig_f32(means3D, "means3D")
    L.check(L.lib().nest_build_homotrans(P, L.ptr(rot), L.ptr(sc), L.ptr(mn), L.ptr(out),
                                         L.stream_ptr(rotations.device)), "nest_build_homotrans")
    return out


def mark_visible(means3D: torch.Tensor, viewmatrix) -> torch.Tensor:
    """markVisible (DSR/rasterize_points.cu:452-470): bool [P], True where the
    view-space depth of the point exceeds 0.2."""
    if means3D.ndim != 2 or means3D.shape[1] != 3:
        raise ValueError("means3D must have dimensions (num_points, 3)")
    P = int(means3D.shape[0])
    present = torch.zeros((P,), dtype=torch.bool, device=means3D.device)
    if P == 0:
        return present
    means3D = _contig_f32(means3D, "means3D")
    vm = host_array(viewmatrix, np.float32)
    if vm.size != 16:
        raise ValueError("viewmatrix must have 16 elements")
    view = (ct.c_float * 16)(*[float(v) for v in vm])
    L.check(L.lib().nest_mark_visible(P, L.ptr(means3D), view, L.ptr(present), L.stream_ptr(means3D.device)),
            "nest_mark_visible")
    return present


def binning_arrays(res: ForwardResult, W: int, H: int) -> Dict[str, torch.Tensor]:
    """Views of the frame's workspaces; the sorted keys (the reference's
    point_list_keys) are composed on this call (nest_binning_keys)."""
    NR = res.num_rendered
    P = int(res.radii.shape[0])
    L.check(L.lib().nest_binning_keys(W, H, P, L.ptr(res.geom), res.geom.numel() * res.geom.element_size(),
                                      L.ptr(res.binning), res.binning.numel() * res.binning.element_size(),
                                      L.ptr(res.image), res.image.numel() * res.image.element_size(), NR,
                                      L.stream_ptr(res.geom.device)), "nest_binning_keys")
    n = max(NR, 1)
    o, _ = L.binning_layout(NR)
    io, _ = L.image_layout(W, H)
    tiles = ((W + 15) // 16) * ((H + 15) // 16)
    return dict(pair_tiles=L.view(res.binning, o[L.BIN_PAIR_TILES], torch.int32, (n,))[:NR],
                pair_ids=L.view(res.binning, o[L.BIN_PAIR_IDS], torch.int32, (n,))[:NR],
                keys=L.view(res.binning, o[L.BIN_KEYS], torch.int64, (n,))[:NR],
                vals=L.view(res.binning, o[L.BIN_VALS], torch.int32, (n,))[:NR],
                ranges=L.view(res.image, io[L.IMG_RANGES], torch.int32, (tiles, 2)),
                final_T=L.view(res.image, io[L.IMG_FINAL_T], torch.float32, (3, H, W)),
                n_contrib=L.view(res.image, io[L.IMG_N_CONTRIB], torch.int32, (2, H, W)),
                tile_order=L.view(res.image, io[L.IMG_TILE_ORDER], torch.int32, (tiles,)))
