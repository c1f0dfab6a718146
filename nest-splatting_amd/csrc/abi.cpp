// C ABI of the forward renderer: argument validation, workspace layout,
// stage sequencing on the caller's stream.
//
// Host orchestration counterpart of CudaRasterizer::Rasterizer::forward
// (submodules/diff-surfel-rasterization/cuda_rasterizer/rasterizer_impl.cu:
// 255-440) and RasterizeGaussiansCUDA (submodules/diff-surfel-rasterization/
// rasterize_points.cu:40-242).  Differences by design: every launch goes to
// the caller's stream instead of the legacy default stream, the library never
// allocates (workspaces come from the caller), the hash-grid offsets and grid
// range arrive as host values instead of device tensors read with .item(), and
// an unsupported configuration is an error instead of a printf and zeros.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/nest_splat.h"
#include "nest_internal.h"

using namespace nest;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(NEST_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

size_t align_up(size_t v, size_t a = 256) { return (v + a - 1) / a * a; }

// Sequential carving of one workspace into 256-byte aligned arrays.
struct Carver {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes);
    return o;
  }
};

uint32_t higher_msb(uint32_t n) {  // getHigherMsb, rasterizer_impl.cu:35-50
  uint32_t msb = sizeof(n) * 4;
  uint32_t step = msb;
  while (step > 1) {
    step /= 2;
    if (n >> msb) msb += step;
    else msb -= step;
  }
  if (n >> msb) msb++;
  return msb;
}

// Per-level constants of query_feature / kernel_grid (hashgrid.h:122-131,
// gridencoder.cu:130-132) and the outcome of get_grid_index's uint32 stride
// loop (hashgrid.h:22-40) for D dimensions.
int build_levels(const int32_t* offsets, uint32_t L, float S, uint32_t H, bool align_corners, int D, bool hash_type,
                 LevelTable& lv) {
  if (L > NEST_MAX_LEVELS) return fail(NEST_ERR_UNSUPPORTED, "at most %d hash levels are supported (got %u)", NEST_MAX_LEVELS, L);
  memset(&lv, 0, sizeof(lv));
  for (uint32_t l = 0; l < L; l++) {
    if (offsets[l] < 0 || offsets[l + 1] <= offsets[l])
      return fail(NEST_ERR_INVALID_ARGUMENT, "hash-grid offsets must be non-negative and strictly increasing (level %u)", l);
    const uint32_t hsize = (uint32_t)(offsets[l + 1] - offsets[l]);
    const float e = (float)l * S;
    const float scale = (float)std::exp2((double)e) * (float)H - 1.0f;
    const uint32_t res = (uint32_t)std::ceil(scale) + 1u;
    const uint32_t res1 = align_corners ? res : res + 1u;
    uint32_t stride = 1, ndims = 0;
    for (int d = 0; d < D && stride <= hsize; d++) {
      ndims++;
      stride *= res1;
    }
    const bool hashed = hash_type && stride > hsize;
    uint64_t bound = 0, st = 1;
    for (uint32_t d = 0; d < ndims; d++) {
      bound += (uint64_t)res * st;
      st *= res1;
    }
    uint32_t flags = 0;
    if (hashed) flags |= 1u;
    if ((hsize & (hsize - 1u)) == 0) flags |= 2u;
    if (!hashed && bound < hsize) flags |= 4u;
    flags |= ndims << 8;
    lv.scale[l] = scale;
    lv.res1[l] = res1;
    lv.hsize[l] = hsize;
    lv.base[l] = (uint32_t)offsets[l];
    lv.flags[l] = flags;
  }
  return NEST_OK;
}

// Records a start/stop event pair per stage into the caller's nest_timing;
// nothing waits here, nest_timing_read() collects the times later.
struct StageTimer {
  nest_timing* t;
  hipStream_t s;
  int stage = -1;
  StageTimer(nest_timing* t_, hipStream_t s_) : t(t_ && t_->enabled ? t_ : nullptr), s(s_) {}
  void begin(int st) {
    if (!t || st < 0 || st >= NEST_STAGE_COUNT) return;
    stage = st;
    for (int k = 0; k < 2; k++) {
      void*& ev = t->events[2 * st + k];
      if (!ev) {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) {
          stage = -1;
          return;
        }
        ev = e;
      }
    }
    hipEventRecord(static_cast<hipEvent_t>(t->events[2 * st]), s);
  }
  void end() {
    if (!t || stage < 0) return;
    hipEventRecord(static_cast<hipEvent_t>(t->events[2 * stage + 1]), s);
    t->recorded |= 1u << stage;
    stage = -1;
  }
};

int check_stage(hipError_t e, const char* what, bool debug, hipStream_t s) {
  if (e != hipSuccess) return hip_fail(e, what);
  if (debug) {
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, what);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
  }
  return NEST_OK;
}

int check_settings(const nest_raster_settings* rs) {
  if (!rs) return fail(NEST_ERR_INVALID_ARGUMENT, "settings is NULL");
  if (rs->struct_size != sizeof(nest_raster_settings))
    return fail(NEST_ERR_INVALID_ARGUMENT, "nest_raster_settings.struct_size is %u, expected %zu", rs->struct_size,
                sizeof(nest_raster_settings));
  if (rs->image_width <= 0 || rs->image_height <= 0)
    return fail(NEST_ERR_INVALID_ARGUMENT, "image size must be positive (got %dx%d)", rs->image_width, rs->image_height);
  if ((int64_t)rs->image_width * rs->image_height > (int64_t)1 << 31)
    return fail(NEST_ERR_UNSUPPORTED, "image has more than 2^31 pixels");
  return NEST_OK;
}

int check_splats(const nest_splats* sp, bool need_geometry) {
  if (!sp) return fail(NEST_ERR_INVALID_ARGUMENT, "splats is NULL");
  if (sp->struct_size != sizeof(nest_splats))
    return fail(NEST_ERR_INVALID_ARGUMENT, "nest_splats.struct_size is %u, expected %zu", sp->struct_size, sizeof(nest_splats));
  if (sp->P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0 (got %d)", sp->P);
  if (need_geometry && sp->P > 0 && (!sp->means3D || !sp->scales || !sp->rotations || !sp->opacities))
    return fail(NEST_ERR_INVALID_ARGUMENT, "means3D, scales, rotations and opacities are required");
  if (sp->kernel_type < 0 || sp->kernel_type > 3)
    return fail(NEST_ERR_UNSUPPORTED, "kernel_type %d: supported are 0 (Gaussian), 1 (beta), 2 (flex), 3 (general)",
                sp->kernel_type);
  if (sp->kernel_type != 0 && sp->P > 0 && !sp->shapes)
    return fail(NEST_ERR_INVALID_ARGUMENT, "kernel_type %d needs shapes [P]", sp->kernel_type);
  if (sp->shs && !sp->colors_precomp) {
    if (sp->sh_degree < 0 || sp->sh_degree > 3)
      return fail(NEST_ERR_UNSUPPORTED, "SH degree must be 0..3 (got %d)", sp->sh_degree);
    if (sp->sh_coeffs < (sp->sh_degree + 1) * (sp->sh_degree + 1))
      return fail(NEST_ERR_INVALID_ARGUMENT, "%d SH coefficients per splat cannot hold degree %d", sp->sh_coeffs,
                  sp->sh_degree);
  }
  return NEST_OK;
}

// SH colours are evaluated when SH coefficients come without precomputed
// colours (CR/forward.cu:417-424).
bool sh_colours(const nest_splats* sp) { return sp->shs && !sp->colors_precomp; }

// Validates the hash-grid settings (or, for levels == 0, the colour inputs)
// for a render with `channels` output channels and fills g (shared by the
// forward render and its backward).
int setup_grid(const nest_raster_settings* rs, const nest_hashgrid* gr, const nest_splats* sp, int channels,
               GridParams& g) {
  int rc = NEST_OK;
  const int base_mode = gr->render_mode & 0xFF;
  const bool adaptive = base_mode == NEST_MODE_ADAPTIVE_CAT || base_mode == NEST_MODE_ADAPTIVE_CAT_FAST ||
                        base_mode == NEST_MODE_ADAPTIVE_ZERO;
  const bool hsh = base_mode >= NEST_MODE_HYBRID_SH && base_mode <= NEST_MODE_HYBRID_SH_RAW;
  const bool dual = base_mode == NEST_MODE_BASELINE_DOUBLE || base_mode == NEST_MODE_BASELINE_BLEND_DOUBLE;
  const bool surf = base_mode == NEST_MODE_SURFACE || base_mode == NEST_MODE_SURFACE_RGB;
  if ((gr->render_mode & ~0x1FF) != 0 ||
      (base_mode != NEST_MODE_BASELINE && base_mode != NEST_MODE_CAT && base_mode != NEST_MODE_ADAPTIVE_ADD &&
       base_mode != NEST_MODE_ADAPTIVE && !adaptive && !hsh && !dual && !surf) ||
      ((gr->render_mode & NEST_MODE_INFERENCE) && !adaptive))
    return fail(NEST_ERR_UNSUPPORTED,
                "render_mode %d: supported are 0-10, 12, 13, 14 and 12, 13, 14 | 0x100", gr->render_mode);
  const bool mix = base_mode != NEST_MODE_BASELINE && !hsh && !dual && !surf;
  if (surf) {
    // surface potentials: F = 12 (mode 1) or 15 (mode 5) features per level,
    // float32 (CR/forward.cu:1825-1908)
    const uint32_t F = base_mode == NEST_MODE_SURFACE ? 12u : 15u, per = base_mode == NEST_MODE_SURFACE ? 4u : 7u;
    if (gr->levels == 0 || gr->level_dim != F || gr->table_dtype != NEST_DTYPE_F32)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d needs float32 grid levels with level_dim %u", base_mode, F);
    if (per * gr->levels > 64u)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d: at most 64 feature channels (got %u)", base_mode,
                  per * gr->levels);
    if ((uint32_t)channels < per * gr->levels)
      return fail(NEST_ERR_INVALID_ARGUMENT, "out_color has %d channels, render_mode %d produces %u", channels,
                  base_mode, per * gr->levels);
    if (base_mode == NEST_MODE_SURFACE && gr->table2) {
      if (gr->offsets2[gr->levels] > gr->table2_rows)
        return fail(NEST_ERR_INVALID_ARGUMENT, "second table has %lld rows, offsets2[%u] = %d",
                    (long long)gr->table2_rows, gr->levels, gr->offsets2[gr->levels]);
      if (!(gr->gridrange2[1] > gr->gridrange2[0]))
        return fail(NEST_ERR_INVALID_ARGUMENT, "gridrange2 must satisfy min < max");
    }
    if (sp->P > 0) {
      if (!sp->homotrans) return fail(NEST_ERR_INVALID_ARGUMENT, "homotrans is required in render_mode %d", base_mode);
      if (!gr->rows2)
        return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode %d needs rows2, a [P, levels * 4] float scratch", base_mode);
    }
  }
  if (dual) {
    // a second grid at the splat centres, 4 features per level in both
    // (CR/forward.cu:1146-1217)
    if (gr->levels == 0 || gr->level_dim != 4)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d needs grid levels with level_dim 4 (got %u levels of %u)",
                  base_mode, gr->levels, gr->level_dim);
    const uint32_t feat = (base_mode == NEST_MODE_BASELINE_DOUBLE ? 2u : 1u) * gr->levels * 4u;
    if (feat > 64u)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d: at most 64 feature channels (got %u)", base_mode, feat);
    if ((uint32_t)channels < feat)
      return fail(NEST_ERR_INVALID_ARGUMENT, "out_color has %d channels, render_mode %d produces %u", channels,
                  base_mode, feat);
    if (gr->table2) {
      if (gr->offsets2[gr->levels] > gr->table2_rows)
        return fail(NEST_ERR_INVALID_ARGUMENT, "second table has %lld rows, offsets2[%u] = %d",
                    (long long)gr->table2_rows, gr->levels, gr->offsets2[gr->levels]);
      if (!(gr->gridrange2[1] > gr->gridrange2[0]))
        return fail(NEST_ERR_INVALID_ARGUMENT, "gridrange2 must satisfy min < max");
    }
    if (sp->P > 0) {
      if (!sp->homotrans) return fail(NEST_ERR_INVALID_ARGUMENT, "homotrans is required in render_mode %d", base_mode);
      if (!gr->rows2)
        return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode %d needs rows2, a [P, levels * 4] float scratch", base_mode);
    }
  }
  if (hsh) {
    // one 3-channel float32 grid level and rows of 3 raw colours or 48 SH
    // coefficients (CR/forward.cu:1378-1542)
    if (gr->levels > 1)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d looks up one grid level (levels must be 0 or 1, got %u)",
                  base_mode, gr->levels);
    if (gr->levels == 1 && (gr->level_dim != 3 || gr->table_dtype != NEST_DTYPE_F32))
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d needs a float32 grid with level_dim 3", base_mode);
    if (gr->decompose > 2)
      return fail(NEST_ERR_INVALID_ARGUMENT, "decompose must be 0, 1 or 2 (got %u)", gr->decompose);
    const int need = base_mode == NEST_MODE_HYBRID_SH_POST ? 48 : 3;
    if (channels < need)
      return fail(NEST_ERR_INVALID_ARGUMENT, "out_color has %d channels, render_mode %d produces %d", channels,
                  base_mode, need);
    if (sp->P > 0) {
      if (!sp->homotrans) return fail(NEST_ERR_INVALID_ARGUMENT, "homotrans is required in render_mode %d", base_mode);
      if (!sp->colors_precomp)
        return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode %d needs the per-splat rows (%d floats) in colors_precomp",
                    base_mode, need);
    }
  }
  if (mix) {
    const uint32_t F = gr->level_dim, hyb = gr->hybrid_levels;
    if (F != 2 && F != 4 && F != 8)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d needs level_dim 2, 4 or 8 (got %u)", gr->render_mode, F);
    if (gr->levels > NEST_MAX_LEVELS || hyb > NEST_MAX_LEVELS || gr->total_levels > NEST_MAX_LEVELS)
      return fail(NEST_ERR_UNSUPPORTED, "levels, hybrid_levels and total_levels must be <= %d", NEST_MAX_LEVELS);
    uint32_t feat = 0;
    if (base_mode == NEST_MODE_ADAPTIVE_ADD && hyb != 0)
      return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode 7 has no per-splat coarse levels (hybrid_levels must be 0)");
    if (base_mode == NEST_MODE_ADAPTIVE && hyb != 0)
      return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode 6 has no per-splat coarse levels (hybrid_levels must be 0)");
    if (base_mode == NEST_MODE_CAT) {
      feat = (hyb + gr->levels) * F;
    } else if (base_mode == NEST_MODE_ADAPTIVE) {
      feat = gr->levels * F;
    } else {
      if (hyb + gr->levels > gr->total_levels)
        return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode %d: hybrid_levels + levels (%u + %u) exceed total_levels %u",
                    base_mode, hyb, gr->levels, gr->total_levels);
      feat = gr->total_levels * F;
    }
    if (feat > 64u)
      return fail(NEST_ERR_UNSUPPORTED, "render_mode %d: at most 64 feature channels (got %u)", gr->render_mode, feat);
    if ((uint32_t)channels < feat)
      return fail(NEST_ERR_INVALID_ARGUMENT, "out_color has %d channels, render_mode %d produces %u", channels,
                  gr->render_mode, feat);
    if (sp->P > 0) {
      if (!sp->homotrans) return fail(NEST_ERR_INVALID_ARGUMENT, "homotrans is required in render_mode %d", gr->render_mode);
      if (!sp->colors_precomp &&
          (adaptive || base_mode == NEST_MODE_ADAPTIVE_ADD || base_mode == NEST_MODE_ADAPTIVE || hyb > 0))
        return fail(NEST_ERR_INVALID_ARGUMENT, "render_mode %d needs the per-splat features in colors_precomp",
                    gr->render_mode);
      // the render queue packs the splat id into 25 bits
      if (sp->P >= (1 << 25))
        return fail(NEST_ERR_UNSUPPORTED, "render_mode %d: at most %d splats", gr->render_mode, (1 << 25) - 1);
    }
    g.F = F;
  }
  if (gr->levels > 0) {
    if (!hsh && !surf && gr->level_dim != 1 && gr->level_dim != 2 && gr->level_dim != 4 && gr->level_dim != 8)
      return fail(NEST_ERR_UNSUPPORTED, "level_dim must be 1, 2, 4 or 8 (got %u)", gr->level_dim);
    if (gr->levels > NEST_MAX_LEVELS || (!surf && gr->levels * gr->level_dim > NEST_MAX_CHANNELS))
      return fail(NEST_ERR_UNSUPPORTED, "levels*level_dim must be <= %d (got %u*%u)", NEST_MAX_CHANNELS, gr->levels,
                  gr->level_dim);
    if (!surf && (uint32_t)channels < gr->levels * gr->level_dim)
      return fail(NEST_ERR_INVALID_ARGUMENT, "out_color has %d channels, the hash grid produces %u", channels,
                  gr->levels * gr->level_dim);
    if (gr->table_dtype != NEST_DTYPE_F32 && gr->table_dtype != NEST_DTYPE_F16)
      return fail(NEST_ERR_UNSUPPORTED, "hash table dtype must be float32 or float16");
    if (gr->interpolation != 0 && gr->interpolation != 1)
      return fail(NEST_ERR_UNSUPPORTED, "interpolation must be 0 (linear) or 1 (smoothstep)");
    if (!gr->table) return fail(NEST_ERR_INVALID_ARGUMENT, "hash table pointer is NULL");
    if (gr->offsets[gr->levels] > gr->table_rows)
      return fail(NEST_ERR_INVALID_ARGUMENT, "hash table has %lld rows, offsets[%u] = %d", (long long)gr->table_rows,
                  gr->levels, gr->offsets[gr->levels]);
    if (!(gr->gridrange[1] > gr->gridrange[0])) return fail(NEST_ERR_INVALID_ARGUMENT, "gridrange must satisfy min < max");
    if (sp->P > 0 && !sp->homotrans) return fail(NEST_ERR_INVALID_ARGUMENT, "homotrans is required on the hash path");
    if ((rc = build_levels(gr->offsets, gr->levels, gr->log2_scale, gr->base_resolution, gr->align_corners != 0, 3, true,
                           g.lv)))
      return rc;
    g.L = gr->levels;
    g.F = gr->level_dim;
    g.interp = (uint32_t)gr->interpolation;
    g.contract = rs->if_contract ? 1u : 0u;
    g.vmin = gr->gridrange[0];
    g.vmax = gr->gridrange[1];
    if (!g.contract) {
      g.inv_size = 1.0f / (g.vmax - g.vmin);
      g.vmid = 0.0f;
    } else {
      g.vmid = (g.vmax + g.vmin) * 0.5f;
      g.inv_size = 1.0f / ((g.vmax - g.vmin) * 0.5f);
    }
    g.pos_offset = gr->align_corners ? 0.0f : 0.5f;
    g.half = gr->table_dtype == NEST_DTYPE_F16 ? 1u : 0u;
    g.table = gr->table;
    const uint64_t tbytes = (uint64_t)gr->table_rows * gr->level_dim * (g.half ? 2u : 4u);
    if (tbytes >= (1ull << 32))
      return fail(NEST_ERR_UNSUPPORTED, "hash table of %llu bytes: at most 4 GiB (32-bit buffer offsets)",
                  (unsigned long long)tbytes);
    g.table_bytes = (uint32_t)tbytes;
    g.table_rows = (uint32_t)gr->table_rows;
    // structured grid: a prefix of dense levels without modulo, then hashed
    // levels with power-of-two sizes (flag bits: 1 hashed, 2 pow2, 4 nomod),
    // trilinear interpolation, cell positions offset by 0.5 (its cell
    // fraction is fract(x), exact for x >= 0: with the 0.5 offset x stays
    // positive even for a grid coordinate that rounds a few ulp below 0;
    // align_corners grids take the general path's x - floor(x))
    uint32_t nd = 0;
    while (nd < g.L && (g.lv.flags[nd] & 5u) == 4u) nd++;
    bool structured = g.interp == 0 && !gr->align_corners;
    for (uint32_t l = nd; l < g.L; l++) structured = structured && (g.lv.flags[l] & 3u) == 3u;
    g.structured = structured ? 1u : 0u;
    g.n_dense = nd;
  } else if (!mix) {
    if (sp->P > 0 && !sp->colors_precomp && !sp->shs)
      return fail(NEST_ERR_INVALID_ARGUMENT, "levels == 0 selects the colour path, which needs colors_precomp or shs");
    // SH colours are RGB (NUM_CHANNELS, CR/rasterizer_impl.cu:320-323)
    if (sh_colours(sp) && channels != 3)
      return fail(NEST_ERR_INVALID_ARGUMENT, "colours from SH have 3 channels, out_color has %d", channels);
  }
  return NEST_OK;
}

}  // namespace

extern "C" {

int nest_abi_version(void) { return NEST_ABI_VERSION; }

const char* nest_last_error(void) { return g_last_error.c_str(); }

int nest_geom_layout(int32_t P, size_t offsets[NEST_GEOM_FIELDS], size_t* total) {
  if (P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0");
  const size_t n = (size_t)(P > 0 ? P : 1);
  Carver c;
  size_t o[NEST_GEOM_FIELDS];
  o[NEST_GEOM_DEPTH] = c.take(n * 4);
  o[NEST_GEOM_XY] = c.take(n * 8);
  o[NEST_GEOM_TILES] = c.take(n * 4);
  o[NEST_GEOM_OFFSETS] = c.take(n * 4);
  o[NEST_GEOM_RECORDS] = c.take(n * kRecordFloats * 4);
  o[NEST_GEOM_RADII] = c.take(n * 4);
  o[NEST_GEOM_SCAN_TMP] = c.take(scan_ws_bytes((int64_t)n));
  o[NEST_GEOM_DEPTH_ORDER] = c.take(n * 4);
  o[NEST_GEOM_ORDER_OFFSETS] = c.take(n * 4);
  o[NEST_GEOM_ORDER_TMP] = c.take(depth_order_ws_bytes((int)n));
  o[NEST_GEOM_RGB] = c.take(n * 12);
  o[NEST_GEOM_CLAMPED] = c.take(n * 3);
  o[NEST_GEOM_RECT] = c.take(n * 8);
  o[NEST_GEOM_ORDER_RECT] = c.take(n * 8);
  if (offsets)
    for (int i = 0; i < NEST_GEOM_FIELDS; i++) offsets[i] = o[i];
  if (total) *total = c.off;
  return NEST_OK;
}

int nest_binning_layout(int64_t NR, size_t offsets[NEST_BIN_FIELDS], size_t* total) {
  if (NR < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "num_rendered must be >= 0");
  const size_t n = (size_t)(NR > 0 ? NR : 1);
  Carver c;
  size_t o[NEST_BIN_FIELDS];
  o[NEST_BIN_PAIR_TILES] = c.take(n * 4);
  o[NEST_BIN_PAIR_IDS] = c.take(n * 4);
  o[NEST_BIN_KEYS] = c.take(n * 8);
  o[NEST_BIN_VALS] = c.take(n * 4);
  o[NEST_BIN_SORT_TMP] = c.take(tile_sort_ws_bytes((int64_t)n));
  if (offsets)
    for (int i = 0; i < NEST_BIN_FIELDS; i++) offsets[i] = o[i];
  if (total) *total = c.off;
  return NEST_OK;
}

int nest_image_layout(int32_t W, int32_t H, size_t offsets[NEST_IMG_FIELDS], size_t* total) {
  if (W <= 0 || H <= 0) return fail(NEST_ERR_INVALID_ARGUMENT, "image size must be positive");
  const size_t tiles = (size_t)((W + kTile - 1) / kTile) * (size_t)((H + kTile - 1) / kTile);
  const size_t HW = (size_t)W * H;
  Carver c;
  size_t o[NEST_IMG_FIELDS];
  o[NEST_IMG_RANGES] = c.take(tiles * 8);
  o[NEST_IMG_FINAL_T] = c.take(HW * 3 * 4);
  o[NEST_IMG_N_CONTRIB] = c.take(HW * 2 * 4);
  o[NEST_IMG_LEVELS] = c.take(sizeof(LevelQuad) * NEST_MAX_LEVELS);
  o[NEST_IMG_TILE_ORDER] = c.take(tiles * 4);
  if (offsets)
    for (int i = 0; i < NEST_IMG_FIELDS; i++) offsets[i] = o[i];
  if (total) *total = c.off;
  return NEST_OK;
}

int nest_hashgrid_levels(const nest_hashgrid* gr, float* scale, uint32_t* resolution, uint32_t* hashed) {
  if (!gr || gr->struct_size < sizeof(nest_hashgrid)) return fail(NEST_ERR_INVALID_ARGUMENT, "grid struct is missing or too small");
  if (gr->levels == 0) return NEST_OK;
  LevelTable lv;
  const int rc = build_levels(gr->offsets, gr->levels, gr->log2_scale, gr->base_resolution, gr->align_corners != 0, 3,
                              true, lv);
  if (rc) return rc;
  for (uint32_t l = 0; l < gr->levels; l++) {
    if (scale) scale[l] = lv.scale[l];
    // res1 is resolution (align_corners) or resolution + 1
    if (resolution) resolution[l] = gr->align_corners ? lv.res1[l] : lv.res1[l] - 1u;
    if (hashed) hashed[l] = lv.flags[l] & 1u;
  }
  return NEST_OK;
}

int nest_forward_geometry(const nest_raster_settings* rs, const nest_splats* sp, void* geom_ws, size_t geom_bytes,
                          int32_t* radii, int64_t* num_rendered, nest_timing* timing, void* stream) {
  int rc = check_settings(rs);
  if (rc) return rc;
  if ((rc = check_splats(sp, true))) return rc;
  if (!num_rendered) return fail(NEST_ERR_INVALID_ARGUMENT, "num_rendered is NULL");
  if (rs->prefiltered) return fail(NEST_ERR_UNSUPPORTED, "prefiltered=True is not supported");
  size_t off[NEST_GEOM_FIELDS], need = 0;
  nest_geom_layout(sp->P, off, &need);
  if (!geom_ws || geom_bytes < need)
    return fail(NEST_ERR_WORKSPACE, "geometry workspace too small: %zu bytes given, %zu needed", geom_bytes, need);
  *num_rendered = 0;
  if (sp->P == 0) return NEST_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* g = static_cast<char*>(geom_ws);
  const int W = rs->image_width, H = rs->image_height;

  PreprocessParams p{};
  p.P = sp->P;
  p.W = W;
  p.H = H;
  p.gx = (uint32_t)((W + kTile - 1) / kTile);
  p.gy = (uint32_t)((H + kTile - 1) / kTile);
  // tile rectangles pack 16-bit tile coordinates
  if (p.gx > 0xFFFFu || p.gy > 0xFFFFu)
    return fail(NEST_ERR_UNSUPPORTED, "image of %d x %d pixels: at most 65535 tiles per side", W, H);
  p.scale_mod = rs->scale_modifier;
  p.beta = rs->beta;
  memcpy(p.view, rs->viewmatrix, sizeof(p.view));
  memcpy(p.proj, rs->projmatrix, sizeof(p.proj));
  p.means = sp->means3D;
  p.scales = sp->scales;
  p.rots = sp->rotations;
  p.opac = sp->opacities;
  p.homotrans = sp->homotrans;
  p.ap_level = sp->ap_level;
  p.kernel_type = sp->kernel_type;
  p.shapes = sp->shapes;
  p.radii = reinterpret_cast<int32_t*>(g + off[NEST_GEOM_RADII]);
  p.radii_user = radii;
  p.xy = reinterpret_cast<float*>(g + off[NEST_GEOM_XY]);
  p.depth = reinterpret_cast<float*>(g + off[NEST_GEOM_DEPTH]);
  p.tiles = reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_TILES]);
  p.rect = reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_RECT]);
  p.depth_key = reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_ORDER_TMP]);  // the depth sort's input keys
  p.records = reinterpret_cast<float*>(g + off[NEST_GEOM_RECORDS]);
  if (sh_colours(sp)) {
    p.shs = sp->shs;
    p.sh_degree = sp->sh_degree;
    p.sh_coeffs = sp->sh_coeffs;
    memcpy(p.campos, rs->campos, sizeof(p.campos));
    p.rgb = reinterpret_cast<float*>(g + off[NEST_GEOM_RGB]);
    p.clamped = reinterpret_cast<uint8_t*>(g + off[NEST_GEOM_CLAMPED]);
  }

  StageTimer tm(timing, s);
  tm.begin(NEST_STAGE_PREPROCESS);
  if ((rc = check_stage(launch_preprocess(p, s), "preprocess", rs->debug, s))) return rc;
  tm.end();
  tm.begin(NEST_STAGE_SCAN);
  uint32_t* offs = reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_OFFSETS]);
  void* scan_ws = g + off[NEST_GEOM_SCAN_TMP];
  if ((rc = check_stage(launch_scan_u32(p.tiles, offs, sp->P, scan_ws, s), "scan", rs->debug, s))) return rc;
  tm.end();
  // The scan leaves the 64-bit grand total after the per-block partials.
  const int64_t nb = ((int64_t)sp->P + 4095) / 4096;
  uint64_t total = 0;
  hipError_t e = hipMemcpyAsync(&total, static_cast<uint64_t*>(scan_ws) + nb, sizeof(total), hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return hip_fail(e, "num_rendered read-back");
  hipEvent_t copied = nullptr;
  e = hipEventCreateWithFlags(&copied, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(copied, s);
  if (e != hipSuccess) {
    if (copied) hipEventDestroy(copied);
    return hip_fail(e, "num_rendered read-back");
  }
  // the splats' depth order (it does not depend on the pair count) runs while
  // the host waits for the count and then sizes the binning workspace
  tm.begin(NEST_STAGE_DEPTH_ORDER);
  rc = check_stage(launch_depth_order(sp->P, p.rect,
                                      reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_DEPTH_ORDER]),
                                      reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_ORDER_OFFSETS]),
                                      reinterpret_cast<uint32_t*>(g + off[NEST_GEOM_ORDER_RECT]),
                                      g + off[NEST_GEOM_ORDER_TMP], s),
                   "depth order", rs->debug, s);
  tm.end();
  e = hipEventSynchronize(copied);
  hipEventDestroy(copied);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "num_rendered read-back");
  if (total > 0xffffffffull)
    return fail(NEST_ERR_OVERFLOW, "%llu tile/splat pairs exceed the 32-bit offsets of the binning stage",
                (unsigned long long)total);
  *num_rendered = (int64_t)total;
  return NEST_OK;
}

int nest_forward_render(const nest_raster_settings* rs, const nest_hashgrid* gr, const nest_splats* sp, void* geom_ws,
                        size_t geom_bytes, void* binning_ws, size_t binning_bytes, void* image_ws, size_t image_bytes,
                        int64_t NR, const nest_frame_outputs* out, nest_timing* timing, void* stream) {
  int rc = check_settings(rs);
  if (rc) return rc;
  if ((rc = check_splats(sp, false))) return rc;
  if (!gr || gr->struct_size != sizeof(nest_hashgrid))
    return fail(NEST_ERR_INVALID_ARGUMENT, "nest_hashgrid missing or struct_size mismatch");
  if (!out || out->struct_size != sizeof(nest_frame_outputs))
    return fail(NEST_ERR_INVALID_ARGUMENT, "nest_frame_outputs missing or struct_size mismatch");
  if (!out->out_color || !out->out_others) return fail(NEST_ERR_INVALID_ARGUMENT, "out_color and out_others are required");
  if (out->channels < 1 || out->channels > NEST_MAX_CHANNELS)
    return fail(NEST_ERR_UNSUPPORTED, "out_color channels must be in [1, %d] (got %d)", NEST_MAX_CHANNELS, out->channels);
  if (NR < 0 || NR > 0xffffffffll) return fail(NEST_ERR_INVALID_ARGUMENT, "num_rendered out of range");
  const int W = rs->image_width, H = rs->image_height;
  const uint32_t gx = (uint32_t)((W + kTile - 1) / kTile), gy = (uint32_t)((H + kTile - 1) / kTile);
  const uint32_t ntiles = gx * gy;

  RenderParams rp{};
  rp.W = W;
  rp.H = H;
  rp.gx = gx;
  rp.gy = gy;
  rp.ntiles = ntiles;
  rp.C = out->channels;
  rp.level = (int)gr->levels;
  rp.beta = rs->beta;
  rp.max_intersections = rs->max_intersections;
  rp.kernel_type = sp->kernel_type;
  if ((rc = setup_grid(rs, gr, sp, out->channels, rp.grid))) return rc;
  const int base_mode = gr->render_mode & 0xFF;
  const bool dual = base_mode == NEST_MODE_BASELINE_DOUBLE || base_mode == NEST_MODE_BASELINE_BLEND_DOUBLE;
  const bool surf = base_mode == NEST_MODE_SURFACE || base_mode == NEST_MODE_SURFACE_RGB;
  GridParams grid1 = rp.grid;  // mode 3 looks the first grid up after the render
  if (surf) {
    // surface potentials: the grid's levels at each hit, the centre rows (the
    // second grid's 4 features per level in mode 1, the grid's 3 colours per
    // level in mode 5) in colors
    rp.hsh = base_mode;
    rp.cstride = (int)gr->levels * (base_mode == NEST_MODE_SURFACE ? 4 : 3);
  } else if (dual) {
    // the centre features as per-splat rows ahead of the grid's levels (as in
    // mode 4); mode 2 then writes the grid's channels first, mode 3 blends the
    // rows alone
    rp.mix = 1;
    rp.hyb = (int)gr->levels;
    rp.pgd = rp.hyb * 4;
    rp.cstride = rp.pgd;
    rp.nrow = rp.pgd;
    rp.wslot = -1;
    rp.fthr = INFINITY;
    rp.fneg = 0;
    if (base_mode == NEST_MODE_BASELINE_DOUBLE) {
      rp.rot = rp.pgd;
      rp.rot_n = 2 * rp.pgd;
    } else {
      rp.grid.L = 0;
    }
  } else if (base_mode >= NEST_MODE_HYBRID_SH && base_mode <= NEST_MODE_HYBRID_SH_RAW) {
    // hybrid SH (CR/forward.cu:1378-1542): rows of 3 raw colours or 48 SH coefficients
    rp.hsh = base_mode;
    rp.hsh_dec = (int)gr->decompose;
    rp.cstride = base_mode == NEST_MODE_HYBRID_SH_POST ? 48 : 3;
  } else if (base_mode != NEST_MODE_BASELINE) {
    // per-splat features ahead of the grid's (CR/forward.cu:965-1101, :1218-1282)
    const int F = (int)gr->level_dim;
    rp.mix = 1;
    rp.hyb = (int)gr->hybrid_levels;
    rp.pgd = rp.hyb * F;
    rp.wslot = -1;
    rp.fthr = INFINITY;  // no fast hits unless the mode has an inference or skip rule
    rp.fneg = 0;
    if ((gr->render_mode & 0xFF) == NEST_MODE_CAT) {
      rp.cstride = rp.pgd;
      rp.nrow = rp.pgd;
    } else if ((gr->render_mode & 0xFF) == NEST_MODE_ADAPTIVE) {
      // mode 6 (CR/forward.cu:1283-1325): rows of C floats, the first levels*F
      // channels 0.5 * row + 0.5 * grid; mode 7's blend with a fixed weight
      rp.cstride = out->channels;
      rp.nrow = 0;
      rp.wfix = 0.5f;
      rp.blend = 1;
      rp.nfast = gr->levels;
      rp.nblend = gr->levels;
    } else if ((gr->render_mode & 0xFF) == NEST_MODE_ADAPTIVE_ADD) {
      // mode 7 (CR/forward.cu:1326-1376): rows [total*F | weight], every level
      // weight * row + (1 - weight) * grid, the grid zero past its levels
      const int tdim = (int)gr->total_levels * F;
      rp.cstride = tdim + 1;
      rp.nrow = tdim;
      rp.wslot = tdim;
      rp.blend = 1;
      rp.nfast = gr->total_levels;
      rp.nblend = gr->total_levels;
    } else if ((gr->render_mode & 0xFF) == NEST_MODE_ADAPTIVE_ZERO) {
      // mode 14 (CR/forward.cu:1716-1830): rows [pgd | weight], grid * weight
      rp.cstride = rp.pgd + 1;
      rp.nrow = rp.pgd;
      rp.wslot = rp.pgd;
      rp.infer = (gr->render_mode & NEST_MODE_INFERENCE) ? 1 : 0;
      rp.gscale = 1;
      // skips the grid when !(weight >= 0.1) in inference, !(weight > 1e-6) in training
      rp.fthr = rp.infer ? std::nextafter(0.1f, 0.0f) : 1e-6f;
      rp.fneg = 1;
    } else {
      // modes 12 and 13 (CR/forward.cu:965-1101, :1593-1713)
      const int tdim = (int)gr->total_levels * F;
      const bool m13 = (gr->render_mode & 0xFF) == NEST_MODE_ADAPTIVE_CAT_FAST;
      rp.cstride = tdim + 1;
      rp.nrow = tdim;
      rp.wslot = tdim;
      rp.infer = (gr->render_mode & NEST_MODE_INFERENCE) ? 1 : 0;
      rp.blend = rp.infer ? 0 : 1;
      rp.m13 = m13 ? 1 : 0;
      rp.wcoarse = (m13 && !rp.infer) ? 1 : 0;
      rp.nfast = gr->total_levels - gr->hybrid_levels;
      rp.nblend = gr->levels;
      // inference takes the row when weight > 0.5 (mode 13) or >= 0.9 (mode 12)
      if (rp.infer) rp.fthr = m13 ? 0.5f : std::nextafter(0.9f, 0.0f);
    }
  }

  size_t go[NEST_GEOM_FIELDS], gneed = 0, bo[NEST_BIN_FIELDS], bneed = 0, io[NEST_IMG_FIELDS], ineed = 0;
  nest_geom_layout(sp->P, go, &gneed);
  nest_binning_layout(NR, bo, &bneed);
  nest_image_layout(W, H, io, &ineed);
  if (!geom_ws || geom_bytes < gneed)
    return fail(NEST_ERR_WORKSPACE, "geometry workspace too small: %zu bytes given, %zu needed", geom_bytes, gneed);
  if (NR > 0 && (!binning_ws || binning_bytes < bneed))
    return fail(NEST_ERR_WORKSPACE, "binning workspace too small: %zu bytes given, %zu needed", binning_bytes, bneed);
  if (!image_ws || image_bytes < ineed)
    return fail(NEST_ERR_WORKSPACE, "image workspace too small: %zu bytes given, %zu needed", image_bytes, ineed);

  hipStream_t s = static_cast<hipStream_t>(stream);
  char* g = static_cast<char*>(geom_ws);
  char* b = static_cast<char*>(binning_ws);
  char* im = static_cast<char*>(image_ws);
  uint32_t* ranges = reinterpret_cast<uint32_t*>(im + io[NEST_IMG_RANGES]);
  StageTimer tm(timing, s);

  uint32_t* vals = nullptr;
  if (NR > 0) {
    uint32_t* pair_tiles = reinterpret_cast<uint32_t*>(b + bo[NEST_BIN_PAIR_TILES]);
    uint32_t* pair_ids = reinterpret_cast<uint32_t*>(b + bo[NEST_BIN_PAIR_IDS]);
    vals = reinterpret_cast<uint32_t*>(b + bo[NEST_BIN_VALS]);
    const float* depth = reinterpret_cast<const float*>(g + go[NEST_GEOM_DEPTH]);
    const uint32_t* order = reinterpret_cast<const uint32_t*>(g + go[NEST_GEOM_DEPTH_ORDER]);
    const uint32_t* order_offsets = reinterpret_cast<const uint32_t*>(g + go[NEST_GEOM_ORDER_OFFSETS]);
    const uint32_t* order_rect = reinterpret_cast<const uint32_t*>(g + go[NEST_GEOM_ORDER_RECT]);
    // duplicate stage: the pairs of the splats in the depth order nest_forward_geometry queued
    tm.begin(NEST_STAGE_DUPLICATE);
    rc = check_stage(launch_duplicate_ordered(sp->P, order, order_offsets, order_rect, gx, NR, pair_tiles, pair_ids, s),
                     "duplicate", rs->debug, s);
    if (rc) return rc;
    tm.end();
    tm.begin(NEST_STAGE_SORT);
    const int bit = (int)higher_msb(ntiles);
    // the sorted keys are not needed downstream: nest_binning_keys composes them on request
    rc = check_stage(launch_sort_tiles(pair_tiles, pair_ids, nullptr, vals, NR, bit, depth, ranges, ntiles,
                                       b + bo[NEST_BIN_SORT_TMP], s),
                     "sort", rs->debug, s);
    if (rc) return rc;
    tm.end();
  }
  tm.begin(NEST_STAGE_RANGES);
  if ((rc = check_stage(launch_tile_ranges(ranges, NR, ntiles, s), "tile ranges", rs->debug, s))) return rc;
  tm.end();

  rp.ranges = ranges;
  rp.point_list = vals;
  rp.records = reinterpret_cast<const float*>(g + go[NEST_GEOM_RECORDS]);
  // feature_ptr of CR/rasterizer_impl.cu:399: precomputed colours, else the
  // colours preprocess evaluated from SH
  rp.colors = sh_colours(sp) ? reinterpret_cast<const float*>(g + go[NEST_GEOM_RGB]) : sp->colors_precomp;
  if (dual || surf) rp.colors = gr->rows2;
  rp.out_color = out->out_color;
  rp.out_others = out->out_others;
  rp.final_T = reinterpret_cast<float*>(im + io[NEST_IMG_FINAL_T]);
  rp.n_contrib = reinterpret_cast<uint32_t*>(im + io[NEST_IMG_N_CONTRIB]);
  rp.grid.lq = reinterpret_cast<LevelQuad*>(im + io[NEST_IMG_LEVELS]);
  rp.tile_order = reinterpret_cast<uint32_t*>(im + io[NEST_IMG_TILE_ORDER]);
  if ((out->cover_pixels == nullptr) != (out->trans_avg == nullptr))
    return fail(NEST_ERR_INVALID_ARGUMENT, "cover_pixels and trans_avg are set together or not at all");
  if (out->cover_pixels && sp->P > 0) {
    // record_transmittance: fresh zeros per frame, as the reference allocates them
    hipError_t e = launch_fill_u32(reinterpret_cast<uint32_t*>(out->cover_pixels), 0u, sp->P, s);
    if (e == hipSuccess) e = launch_fill_u32(reinterpret_cast<uint32_t*>(out->trans_avg), 0u, sp->P, s);
    if (e != hipSuccess) return hip_fail(e, "record_transmittance fill");
    rp.cover_pixels = out->cover_pixels;
    rp.trans_avg = out->trans_avg;
  }
  tm.begin(NEST_STAGE_RENDER);
  if (base_mode == NEST_MODE_SURFACE_RGB && sp->P > 0) {
    // the grid's colours at the splat centres (CR/forward.cu:1883-1885)
    hipError_t e = launch_centre_rgb(grid1, sp->P, sp->homotrans, sp->ap_level, gr->rows2, s);
    if (e != hipSuccess) return hip_fail(e, "centre colours");
  }
  if ((dual || base_mode == NEST_MODE_SURFACE) && sp->P > 0) {
    // the second grid's features at the splat centres (CR/forward.cu:1164-1175, :1836-1849)
    hipError_t e = hipSuccess;
    if (gr->table2) {
      GridParams g2 = grid1;
      if ((rc = build_levels(gr->offsets2, gr->levels, gr->log2_scale, gr->base_resolution, gr->align_corners != 0, 3,
                             true, g2.lv)))
        return rc;
      g2.table = gr->table2;
      g2.table_rows = (uint32_t)gr->table2_rows;
      g2.half = 0u;
      g2.vmin = gr->gridrange2[0];
      g2.vmax = gr->gridrange2[1];
      if (!g2.contract) {
        g2.inv_size = 1.0f / (g2.vmax - g2.vmin);
        g2.vmid = 0.0f;
      } else {
        g2.vmid = (g2.vmax + g2.vmin) * 0.5f;
        g2.inv_size = 1.0f / ((g2.vmax - g2.vmin) * 0.5f);
      }
      e = launch_centre_rows(g2, sp->P, sp->homotrans, sp->ap_level, gr->rows2, s);
    } else {
      e = launch_fill_u32(reinterpret_cast<uint32_t*>(gr->rows2), 0u, (int64_t)sp->P * gr->levels * 4, s);
    }
    if (e != hipSuccess) return hip_fail(e, "centre features");
  }
  if ((rc = check_stage(launch_render(rp, s), "render", rs->debug, s))) return rc;
  if (base_mode == NEST_MODE_BASELINE_BLEND_DOUBLE) {
    // the first grid at each pixel's blended position (CR/forward.cu:1975-2004)
    RenderParams ps = rp;
    ps.grid = grid1;
    if ((rc = check_stage(launch_spatial_add(ps, sp->ap_level, s), "blended-position grid", rs->debug, s))) return rc;
  }
  tm.end();
  return NEST_OK;
}

int nest_build_homotrans(int64_t P, const float* rotations, const float* scales, const float* means3D,
                         float* homotrans, void* stream) {
  if (P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0 (got %lld)", (long long)P);
  if (P == 0) return NEST_OK;
  if (!rotations || !scales || !means3D || !homotrans)
    return fail(NEST_ERR_INVALID_ARGUMENT, "rotations, scales, means3D and homotrans are required");
  if ((reinterpret_cast<uintptr_t>(rotations) & 15u) || (reinterpret_cast<uintptr_t>(scales) & 7u) ||
      (reinterpret_cast<uintptr_t>(homotrans) & 15u) || (reinterpret_cast<uintptr_t>(means3D) & 3u))
    return fail(NEST_ERR_INVALID_ARGUMENT, "rotations and homotrans need 16-byte, scales 8-byte alignment");
  hipError_t e = launch_build_homotrans(P, rotations, scales, means3D, homotrans, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "build_homotrans");
}

int nest_mark_visible(int32_t P, const float* means3D, const float viewmatrix[16], uint8_t* present, void* stream) {
  if (P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0 (got %d)", P);
  if (P == 0) return NEST_OK;
  if (!means3D || !viewmatrix || !present)
    return fail(NEST_ERR_INVALID_ARGUMENT, "means3D, viewmatrix and present are required");
  hipError_t e = launch_mark_visible(P, means3D, viewmatrix, present, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "mark_visible");
}

int nest_timing_read(nest_timing* t) {
  if (!t || t->struct_size != sizeof(nest_timing)) return fail(NEST_ERR_INVALID_ARGUMENT, "nest_timing missing or struct_size mismatch");
  for (int st = 0; st < NEST_STAGE_COUNT; st++) {
    t->ms[st] = 0.0f;
    if (!(t->recorded & (1u << st))) continue;
    hipEvent_t a = static_cast<hipEvent_t>(t->events[2 * st]), b = static_cast<hipEvent_t>(t->events[2 * st + 1]);
    hipError_t e = hipEventSynchronize(b);
    if (e != hipSuccess) return hip_fail(e, "nest_timing_read");
    float ms = 0.0f;
    e = hipEventElapsedTime(&ms, a, b);
    if (e != hipSuccess) return hip_fail(e, "nest_timing_read");
    t->ms[st] = ms;
  }
  t->recorded = 0;
  return NEST_OK;
}

int nest_timing_release(nest_timing* t) {
  if (!t || t->struct_size != sizeof(nest_timing)) return fail(NEST_ERR_INVALID_ARGUMENT, "nest_timing missing or struct_size mismatch");
  for (int i = 0; i < 2 * NEST_STAGE_COUNT; i++) {
    if (t->events[i]) hipEventDestroy(static_cast<hipEvent_t>(t->events[i]));
    t->events[i] = nullptr;
  }
  t->recorded = 0;
  return NEST_OK;
}

size_t nest_scan_workspace_size(int64_t n) { return scan_ws_bytes(n > 0 ? n : 1); }

}  // extern "C"

// Scratch of nest_inclusive_scan_u32_noalloc: the scan's block partials,
// (ceil(n / 4096) + 1) 64-bit words, in a device array the library owns.
// Every GPU the library runs on holds its own copy until the process ends;
// the host-side name is only a stand-in, so kernels get the address that
// hipGetSymbolAddress reports for the current device.  The scan writes every
// partial it reads, so nothing has to be cleared between calls.
constexpr size_t kScanScratchBytes = 512u * 1024u;
static __device__ __align__(256) uint64_t scratch[kScanScratchBytes / sizeof(uint64_t)];
static_assert((((int64_t)NEST_SCAN_NOALLOC_MAX + 4095) / 4096 + 1) * 8 <= (int64_t)kScanScratchBytes,
              "NEST_SCAN_NOALLOC_MAX must fit the scratch");

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int scratch_on_current_device(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(NEST_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(NEST_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return NEST_OK;
}

}  // namespace

extern "C" {

int nest_inclusive_scan_u32_noalloc(const uint32_t* in, uint32_t* out, int64_t n, void* stream) {
  if (n < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "n must be >= 0");
  if (n == 0) return NEST_OK;
  if (!in || !out) return fail(NEST_ERR_INVALID_ARGUMENT, "in/out is NULL");
  if (n > (int64_t)NEST_SCAN_NOALLOC_MAX)
    return fail(NEST_ERR_WORKSPACE, "allocation-free scan: n = %lld exceeds the %lld elements its %zu-byte scratch holds",
                (long long)n, (long long)NEST_SCAN_NOALLOC_MAX, kScanScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  hipError_t e = launch_scan_u32(in, out, n, ws, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "scan");
}

int nest_inclusive_scan_u32(const uint32_t* in, uint32_t* out, int64_t n, void* ws, size_t ws_bytes, void* stream) {
  if (n < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "n must be >= 0");
  if (n == 0) return NEST_OK;
  if (!in || !out) return fail(NEST_ERR_INVALID_ARGUMENT, "in/out is NULL");
  if (!ws || ws_bytes < scan_ws_bytes(n))
    return fail(NEST_ERR_WORKSPACE, "scan workspace too small: %zu bytes given, %zu needed", ws_bytes, scan_ws_bytes(n));
  hipError_t e = launch_scan_u32(in, out, n, ws, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "scan");
}

size_t nest_sort_workspace_size(int64_t n) { return sort_ws_bytes(n > 0 ? n : 1); }

int nest_binning_keys(int32_t W, int32_t H, int32_t P, const void* geom_ws, size_t geom_bytes, void* binning_ws,
                      size_t binning_bytes, const void* image_ws, size_t image_bytes, int64_t NR, void* stream) {
  if (W <= 0 || H <= 0) return fail(NEST_ERR_INVALID_ARGUMENT, "image size must be positive");
  if (P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0");
  if (NR < 0 || NR > 0xffffffffll) return fail(NEST_ERR_INVALID_ARGUMENT, "num_rendered out of range");
  size_t go[NEST_GEOM_FIELDS], gneed = 0, bo[NEST_BIN_FIELDS], bneed = 0, io[NEST_IMG_FIELDS], ineed = 0;
  nest_geom_layout(P, go, &gneed);
  nest_binning_layout(NR, bo, &bneed);
  nest_image_layout(W, H, io, &ineed);
  if (!geom_ws || geom_bytes < gneed)
    return fail(NEST_ERR_WORKSPACE, "geometry workspace too small: %zu bytes given, %zu needed", geom_bytes, gneed);
  if (NR > 0 && (!binning_ws || binning_bytes < bneed))
    return fail(NEST_ERR_WORKSPACE, "binning workspace too small: %zu bytes given, %zu needed", binning_bytes, bneed);
  if (!image_ws || image_bytes < ineed)
    return fail(NEST_ERR_WORKSPACE, "image workspace too small: %zu bytes given, %zu needed", image_bytes, ineed);
  if (NR == 0) return NEST_OK;
  const uint32_t ntiles = (uint32_t)(((W + kTile - 1) / kTile) * ((H + kTile - 1) / kTile));
  const char* g = static_cast<const char*>(geom_ws);
  char* b = static_cast<char*>(binning_ws);
  const char* im = static_cast<const char*>(image_ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return check_stage(launch_compose_keys(reinterpret_cast<const uint32_t*>(im + io[NEST_IMG_RANGES]),
                                         reinterpret_cast<const uint32_t*>(b + bo[NEST_BIN_VALS]),
                                         reinterpret_cast<const float*>(g + go[NEST_GEOM_DEPTH]), ntiles,
                                         reinterpret_cast<uint64_t*>(b + bo[NEST_BIN_KEYS]), s),
                     "binning keys", 0, s);
}

int nest_sort_pairs_u64(const uint64_t* keys_in, const uint32_t* vals_in, uint64_t* keys_out, uint32_t* vals_out,
                        int64_t n, int32_t end_bit, void* ws, size_t ws_bytes, void* stream) {
  if (n < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "n must be >= 0");
  if (end_bit < 1 || end_bit > 64) return fail(NEST_ERR_INVALID_ARGUMENT, "end_bit must be in [1, 64]");
  if (n == 0) return NEST_OK;
  if (n > 0xffffffffll) return fail(NEST_ERR_UNSUPPORTED, "at most 2^32-1 pairs");
  if (!keys_in || !vals_in || !keys_out || !vals_out) return fail(NEST_ERR_INVALID_ARGUMENT, "NULL key/value pointer");
  if (!ws || ws_bytes < sort_ws_bytes(n))
    return fail(NEST_ERR_WORKSPACE, "sort workspace too small: %zu bytes given, %zu needed", ws_bytes, sort_ws_bytes(n));
  hipError_t e = launch_sort_pairs(keys_in, vals_in, keys_out, vals_out, n, end_bit, ws, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "sort");
}

int nest_grid_encode(const float* inputs, int64_t B, int32_t D, const void* embeddings, int64_t emb_rows, int32_t emb_dtype,
                     const int32_t* offsets_host, int32_t L, int32_t C, float S, int32_t H, int32_t gridtype,
                     int32_t align_corners, int32_t interpolation, void* outputs, void* stream) {
  if (B < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "B must be >= 0");
  if (D < 2 || D > 5) return fail(NEST_ERR_UNSUPPORTED, "GridEncoding: D must be 2, 3, 4 or 5 (got %d)", D);
  if (C != 1 && C != 2 && C != 4 && C != 8 && C != 16)
    return fail(NEST_ERR_UNSUPPORTED, "GridEncoding: C must be 1, 2, 4, 8 or 16 (got %d)", C);
  if (L < 1 || L > NEST_MAX_LEVELS) return fail(NEST_ERR_UNSUPPORTED, "GridEncoding: L must be in [1, %d]", NEST_MAX_LEVELS);
  if (emb_dtype != NEST_DTYPE_F32 && emb_dtype != NEST_DTYPE_F16)
    return fail(NEST_ERR_UNSUPPORTED, "GridEncoding: embeddings must be float32 or float16");
  if (gridtype != 0 && gridtype != 1) return fail(NEST_ERR_INVALID_ARGUMENT, "gridtype must be 0 (hash) or 1 (tiled)");
  if (interpolation != 0 && interpolation != 1) return fail(NEST_ERR_INVALID_ARGUMENT, "interpolation must be 0 or 1");
  if (!offsets_host) return fail(NEST_ERR_INVALID_ARGUMENT, "offsets is NULL");
  if (offsets_host[L] > emb_rows)
    return fail(NEST_ERR_INVALID_ARGUMENT, "embeddings have %lld rows, offsets[%d] = %d", (long long)emb_rows, L, offsets_host[L]);
  if (B == 0) return NEST_OK;
  if (!inputs || !embeddings || !outputs) return fail(NEST_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  GridEncodeParams p{};
  int rc = build_levels(offsets_host, (uint32_t)L, S, (uint32_t)H, align_corners != 0, D, gridtype == 0, p.lv);
  if (rc) return rc;
  // the common layout (dense prefix without modulo, then power-of-two hashed
  // levels; D = 3, binary32, trilinear) takes the render's lookup
  const uint64_t tbytes = (uint64_t)emb_rows * (uint64_t)C * 4u;
  if (D == 3 && gridtype == 0 && emb_dtype == NEST_DTYPE_F32 && interpolation == 0 && C <= 8 &&
      tbytes < (1ull << 32)) {
    uint32_t nd = 0;
    while (nd < (uint32_t)L && (p.lv.flags[nd] & 5u) == 4u) nd++;
    bool structured = true;
    for (uint32_t l = nd; l < (uint32_t)L; l++) structured = structured && (p.lv.flags[l] & 3u) == 3u;
    if (structured) {
      GridEncodeQuadParams q{};
      q.inputs = inputs;
      q.B = B;
      q.F = C;
      q.L = L;
      q.pos_offset = align_corners ? 0.0f : 0.5f;
      q.table = static_cast<const float*>(embeddings);
      q.table_rows = (uint32_t)emb_rows;
      q.outputs = static_cast<float*>(outputs);
      for (uint32_t l = 0; l < (uint32_t)L; l++) {
        const bool dense = l < nd;
        q.lq[l].scale = p.lv.scale[l];
        q.lq[l].a = dense ? p.lv.res1[l] : p.lv.hsize[l] - 1u;
        q.lq[l].b = dense ? p.lv.res1[l] * p.lv.res1[l] : 0u;
        q.lq[l].soff = p.lv.base[l] * (uint32_t)C * 4u;
      }
      hipError_t e = launch_grid_encode_quad(q, static_cast<hipStream_t>(stream));
      return e == hipSuccess ? NEST_OK : hip_fail(e, "grid_encode");
    }
  }
  p.inputs = inputs;
  p.B = B;
  p.D = D;
  p.C = C;
  p.L = L;
  p.gridtype = gridtype;
  p.align_corners = align_corners;
  p.interp = interpolation;
  p.half = emb_dtype == NEST_DTYPE_F16;
  p.table = embeddings;
  p.outputs = outputs;
  hipError_t e = launch_grid_encode(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "grid_encode");
}

int nest_grid_encode_backward(const float* inputs, int64_t B, int32_t D, const void* embeddings, int64_t emb_rows,
                              int32_t emb_dtype, const int32_t* offsets_host, int32_t L, int32_t C, float S, int32_t H,
                              int32_t gridtype, int32_t align_corners, int32_t interpolation, const float* grad,
                              float* grad_embeddings, float* grad_inputs, void* stream) {
  if (B < 0 || emb_rows < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "B and emb_rows must be >= 0");
  if (D != 3) return fail(NEST_ERR_UNSUPPORTED, "GridEncoding backward: D must be 3 (got %d)", D);
  if (C != 1 && C != 2 && C != 4 && C != 8)
    return fail(NEST_ERR_UNSUPPORTED, "GridEncoding backward: C must be 1, 2, 4 or 8 (got %d)", C);
  if (L < 1 || L > NEST_MAX_LEVELS) return fail(NEST_ERR_UNSUPPORTED, "GridEncoding: L must be in [1, %d]", NEST_MAX_LEVELS);
  if (emb_dtype != NEST_DTYPE_F32) return fail(NEST_ERR_UNSUPPORTED, "GridEncoding backward: embeddings must be float32");
  if (gridtype != 0 && gridtype != 1) return fail(NEST_ERR_INVALID_ARGUMENT, "gridtype must be 0 (hash) or 1 (tiled)");
  if (interpolation != 0 && interpolation != 1) return fail(NEST_ERR_INVALID_ARGUMENT, "interpolation must be 0 or 1");
  if (!offsets_host) return fail(NEST_ERR_INVALID_ARGUMENT, "offsets is NULL");
  if (offsets_host[L] > emb_rows)
    return fail(NEST_ERR_INVALID_ARGUMENT, "embeddings have %lld rows, offsets[%d] = %d", (long long)emb_rows, L, offsets_host[L]);
  if (emb_rows > 0xffffffffll / C) return fail(NEST_ERR_UNSUPPORTED, "embedding table too large");
  if (!grad_embeddings || (B > 0 && (!inputs || !embeddings || !grad)))
    return fail(NEST_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  GridEncodeBwdParams p{};
  int rc = build_levels(offsets_host, (uint32_t)L, S, (uint32_t)H, align_corners != 0, 3, gridtype == 0, p.lv);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = launch_fill_u32(reinterpret_cast<uint32_t*>(grad_embeddings), 0u, emb_rows * C, s);
  if (e != hipSuccess) return hip_fail(e, "grid_encode_backward fill");
  if (B == 0) return NEST_OK;
  p.inputs = inputs;
  p.B = B;
  p.F = C;
  p.L = L;
  p.align_corners = align_corners;
  p.interp = interpolation;
  p.table = static_cast<const float*>(embeddings);
  p.table_rows = (uint32_t)emb_rows;
  p.grad = grad;
  p.grad_table = grad_embeddings;
  p.grad_inputs = grad_inputs;
  e = launch_grid_encode_backward(p, s);
  return e == hipSuccess ? NEST_OK : hip_fail(e, "grid_encode_backward");
}

int nest_backward_layout(int32_t P, int32_t channels, size_t offsets[NEST_BWD_FIELDS], size_t* total) {
  if (P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0");
  if (channels < 1 || channels > NEST_MAX_CHANNELS)
    return fail(NEST_ERR_INVALID_ARGUMENT, "channels must be in [1, %d]", NEST_MAX_CHANNELS);
  const size_t n = (size_t)(P > 0 ? P : 1);
  Carver c;
  size_t o[NEST_BWD_FIELDS];
  o[NEST_BWD_DTRANSMAT] = c.take(n * 9 * 4);
  o[NEST_BWD_DHOMO] = c.take(n * 9 * 4);
  o[NEST_BWD_DNORMAL] = c.take(n * 3 * 4);
  o[NEST_BWD_DCOLORS] = c.take(n * (size_t)channels * 4);
  o[NEST_BWD_GRADSUM] = c.take(n * 4);
  if (offsets)
    for (int i = 0; i < NEST_BWD_FIELDS; i++) offsets[i] = o[i];
  if (total) *total = c.off;
  return NEST_OK;
}

int nest_backward(const nest_raster_settings* rs, const nest_hashgrid* gr, const nest_splats* sp, const void* geom_ws,
                  size_t geom_bytes, const void* binning_ws, size_t binning_bytes, const void* image_ws,
                  size_t image_bytes, int64_t NR, const nest_backward_io* io, void* bwd_ws, size_t bwd_bytes,
                  void* stream) {
  int rc = check_settings(rs);
  if (rc) return rc;
  if ((rc = check_splats(sp, true))) return rc;
  if (!gr || gr->struct_size != sizeof(nest_hashgrid))
    return fail(NEST_ERR_INVALID_ARGUMENT, "nest_hashgrid missing or struct_size mismatch");
  if (!io || io->struct_size != sizeof(nest_backward_io))
    return fail(NEST_ERR_INVALID_ARGUMENT, "nest_backward_io missing or struct_size mismatch");
  if (gr->render_mode != NEST_MODE_BASELINE && gr->render_mode != NEST_MODE_CAT &&
      gr->render_mode != NEST_MODE_ADAPTIVE_ADD && gr->render_mode != NEST_MODE_ADAPTIVE_CAT &&
      gr->render_mode != NEST_MODE_ADAPTIVE_ZERO)
    return fail(NEST_ERR_UNSUPPORTED,
                "backward: render_mode %d is forward-only here (modes 0, 4, 7, 12 and 14 without the inference flag "
                "have a backward)", gr->render_mode);
  const bool cat = gr->render_mode == NEST_MODE_CAT;
  // mode 7 is mode 12 without coarse levels, every level blended
  const bool aadd = gr->render_mode == NEST_MODE_ADAPTIVE_ADD;
  const bool acat = gr->render_mode == NEST_MODE_ADAPTIVE_CAT || aadd;
  const bool azero = gr->render_mode == NEST_MODE_ADAPTIVE_ZERO;
  const int C = io->channels;
  if (C < 1 || C > 64) return fail(NEST_ERR_UNSUPPORTED, "backward: channels must be in [1, 64] (got %d)", C);
  if (!io->dL_dout_color || !io->dL_dout_others)
    return fail(NEST_ERR_INVALID_ARGUMENT, "backward: dL_dout_color and dL_dout_others are required");
  if (sp->kernel_type != 0 && sp->P > 0 && !io->dL_dshapes)
    return fail(NEST_ERR_INVALID_ARGUMENT, "backward: kernel_type %d needs dL_dshapes [P]", sp->kernel_type);
  if (!io->dL_dmeans3D || !io->dL_dmeans2D || !io->dL_dopacity || !io->dL_dscales || !io->dL_drotations)
    return fail(NEST_ERR_INVALID_ARGUMENT, "backward: dL_dmeans3D, dL_dmeans2D, dL_dopacity, dL_dscales and "
                                           "dL_drotations are required");
  if (NR < 0 || NR > 0xffffffffll) return fail(NEST_ERR_INVALID_ARGUMENT, "num_rendered out of range");
  GridParams g{};
  if ((rc = setup_grid(rs, gr, sp, C, g))) return rc;
  const bool hash = gr->levels > 0;
  const bool from_sh = !cat && !acat && !azero && !hash && sh_colours(sp);
  // mode 4: per-splat rows of pgd floats; the grid levels differentiated are
  // those up to the last one within the active count whose offsets increase
  // (CR/backward.cu:576-612, :993-999)
  const int pgd = (cat || acat || azero) ? (int)(gr->hybrid_levels * gr->level_dim) : 0;
  // mode 12: rows of total*F features and the blend weight; the grid's levels
  // are blended (CR/backward.cu:1425-1520)
  const int tdim = acat ? (int)(gr->total_levels * gr->level_dim) : 0;
  uint32_t cat_levels = 0;
  if (cat) {
    const uint32_t act = gr->active_levels < gr->levels ? gr->active_levels : gr->levels;
    for (uint32_t i = 1; i <= act; i++)
      if (gr->offsets[i] > gr->offsets[i - 1]) cat_levels = i;
    g.L = cat_levels;
  }
  const int dcol_width = cat ? pgd : acat ? tdim + 1 : azero ? pgd + 1 : C;
  // the workspace's colour-gradient field holds [P, channels]: mode-12 rows are wider
  if ((acat || azero) && !io->dL_dcolors)
    return fail(NEST_ERR_INVALID_ARGUMENT, "backward: render_mode %d needs dL_dcolors [P, %d]", gr->render_mode,
                dcol_width);
  if (hash && g.half) return fail(NEST_ERR_UNSUPPORTED, "backward: the hash table must be float32");
  if (hash && !io->dL_dfeatures) return fail(NEST_ERR_INVALID_ARGUMENT, "backward: dL_dfeatures is required");
  if (from_sh && !io->dL_dshs) return fail(NEST_ERR_INVALID_ARGUMENT, "backward: dL_dshs is required with SH colours");

  const int W = rs->image_width, H = rs->image_height, P = sp->P;
  const uint32_t gx = (uint32_t)((W + kTile - 1) / kTile), gy = (uint32_t)((H + kTile - 1) / kTile);
  size_t go[NEST_GEOM_FIELDS], gneed = 0, bo[NEST_BIN_FIELDS], bneed = 0, io_[NEST_IMG_FIELDS], ineed = 0;
  size_t wo[NEST_BWD_FIELDS], wneed = 0;
  nest_geom_layout(P, go, &gneed);
  nest_binning_layout(NR, bo, &bneed);
  nest_image_layout(W, H, io_, &ineed);
  nest_backward_layout(P, C, wo, &wneed);
  if (!geom_ws || geom_bytes < gneed)
    return fail(NEST_ERR_WORKSPACE, "geometry workspace too small: %zu bytes given, %zu needed", geom_bytes, gneed);
  if (NR > 0 && (!binning_ws || binning_bytes < bneed))
    return fail(NEST_ERR_WORKSPACE, "binning workspace too small: %zu bytes given, %zu needed", binning_bytes, bneed);
  if (!image_ws || image_bytes < ineed)
    return fail(NEST_ERR_WORKSPACE, "image workspace too small: %zu bytes given, %zu needed", image_bytes, ineed);
  if (!bwd_ws || bwd_bytes < wneed)
    return fail(NEST_ERR_WORKSPACE, "backward workspace too small: %zu bytes given, %zu needed", bwd_bytes, wneed);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* gw = static_cast<const char*>(geom_ws);
  const char* im = static_cast<const char*>(image_ws);
  char* bw = static_cast<char*>(bwd_ws);
  float* dtransmat = reinterpret_cast<float*>(bw + wo[NEST_BWD_DTRANSMAT]);
  float* dhomo = reinterpret_cast<float*>(bw + wo[NEST_BWD_DHOMO]);
  float* dnormal = reinterpret_cast<float*>(bw + wo[NEST_BWD_DNORMAL]);
  float* dcolors = io->dL_dcolors ? io->dL_dcolors : reinterpret_cast<float*>(bw + wo[NEST_BWD_DCOLORS]);
  float* gradsum = io->dL_dgradsum ? io->dL_dgradsum : reinterpret_cast<float*>(bw + wo[NEST_BWD_GRADSUM]);
  const int M = from_sh ? sp->sh_coeffs : 0;
  // zero every gradient output and the accumulators
  struct Fill {
    float* p;
    int64_t n;
  } fills[] = {{dtransmat, (int64_t)P * 9}, {dhomo, (int64_t)P * 9}, {dnormal, (int64_t)P * 3},
               {dcolors, (int64_t)P * dcol_width}, {gradsum, (int64_t)P}, {io->dL_dmeans3D, (int64_t)P * 3},
               {io->dL_dmeans2D, (int64_t)P * 3}, {io->dL_dopacity, (int64_t)P}, {io->dL_dscales, (int64_t)P * 2},
               {io->dL_drotations, (int64_t)P * 4}, {from_sh ? io->dL_dshs : nullptr, (int64_t)P * M * 3},
               {hash ? io->dL_dfeatures : nullptr, hash ? (int64_t)gr->table_rows * gr->level_dim : 0},
               {io->dL_dshapes, (int64_t)P}};
  for (const Fill& f : fills) {
    if (!f.p || f.n == 0) continue;
    hipError_t e = launch_fill_u32(reinterpret_cast<uint32_t*>(f.p), 0u, f.n, s);
    if (e != hipSuccess) return hip_fail(e, "backward fill");
  }
  if (P == 0) return NEST_OK;

  RenderBwdParams rp{};
  rp.W = W;
  rp.H = H;
  rp.gx = gx;
  rp.gy = gy;
  rp.ntiles = gx * gy;
  rp.C = C;
  rp.level = (cat || acat || azero) ? 1 : (int)gr->levels;  // these modes always take the hash branch
  rp.pgd = pgd;
  rp.cstride = dcol_width;
  rp.wslot = acat ? tdim : azero ? pgd : -1;
  rp.azero = azero ? 1 : 0;
  rp.nfine = aadd ? tdim : (acat || azero) ? (int)(gr->levels * gr->level_dim) : 0;
  rp.wsig = aadd ? 1 : 0;
  rp.beta = rs->beta;
  rp.ranges = reinterpret_cast<const uint32_t*>(im + io_[NEST_IMG_RANGES]);
  rp.tile_order = reinterpret_cast<const uint32_t*>(im + io_[NEST_IMG_TILE_ORDER]);
  rp.point_list = NR > 0 ? reinterpret_cast<const uint32_t*>(static_cast<const char*>(binning_ws) + bo[NEST_BIN_VALS])
                         : nullptr;
  rp.records = reinterpret_cast<const float*>(gw + go[NEST_GEOM_RECORDS]);
  rp.colors = from_sh ? reinterpret_cast<const float*>(gw + go[NEST_GEOM_RGB]) : sp->colors_precomp;
  rp.final_T = reinterpret_cast<const float*>(im + io_[NEST_IMG_FINAL_T]);
  rp.n_contrib = reinterpret_cast<const uint32_t*>(im + io_[NEST_IMG_N_CONTRIB]);
  rp.dL_dpix = io->dL_dout_color;
  rp.dL_dothers = io->dL_dout_others;
  rp.dtable = hash ? io->dL_dfeatures : nullptr;
  rp.dtransmat = dtransmat;
  rp.dhomo = dhomo;
  rp.dmean2D = io->dL_dmeans2D;
  rp.dnormal = dnormal;
  rp.dopacity = io->dL_dopacity;
  rp.dcolors = dcolors;
  rp.gradsum = gradsum;
  rp.kernel_type = sp->kernel_type;
  rp.dshapes = sp->kernel_type != 0 ? io->dL_dshapes : nullptr;
  rp.grid = g;
  if (NR > 0) {
    hipError_t e = launch_render_backward(rp, s);
    if ((rc = check_stage(e, "render backward", rs->debug, s))) return rc;
  }

  PreprocessBwdParams pp{};
  pp.P = P;
  pp.W = W;
  pp.H = H;
  memcpy(pp.view, rs->viewmatrix, sizeof(pp.view));
  memcpy(pp.proj, rs->projmatrix, sizeof(pp.proj));
  memcpy(pp.campos, rs->campos, sizeof(pp.campos));
  pp.means = sp->means3D;
  pp.scales = sp->scales;
  pp.rots = sp->rotations;
  pp.radii = reinterpret_cast<const int32_t*>(gw + go[NEST_GEOM_RADII]);
  pp.records = reinterpret_cast<const float*>(gw + go[NEST_GEOM_RECORDS]);
  pp.shs = from_sh ? sp->shs : nullptr;
  pp.sh_degree = sp->sh_degree;
  pp.sh_coeffs = M;
  pp.clamped = reinterpret_cast<const uint8_t*>(gw + go[NEST_GEOM_CLAMPED]);
  pp.dcolors = dcolors;
  pp.dtransmat = dtransmat;
  pp.dhomo = dhomo;
  pp.dnormal = dnormal;
  pp.dmean2D = io->dL_dmeans2D;
  pp.dmeans = io->dL_dmeans3D;
  pp.dscales = io->dL_dscales;
  pp.drots = io->dL_drotations;
  pp.dshs = from_sh ? io->dL_dshs : nullptr;
  return check_stage(launch_preprocess_backward(pp, s), "preprocess backward", rs->debug, s);
}

int nest_mlp_decode(const nest_mlp* mlp, const float* feat, int64_t feat_cs, int64_t feat_ns, int64_t N, int32_t width,
                    const float* dirs, const float ray_matrix[9], const float* alpha, const float bg[3], float* out,
                    int64_t out_os, int64_t out_ns, void* stream) {
  if (!mlp || mlp->struct_size != sizeof(nest_mlp)) return fail(NEST_ERR_INVALID_ARGUMENT, "nest_mlp missing or struct_size mismatch");
  if (N < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "N must be >= 0");
  if (mlp->in_features < 1 || mlp->in_features > NEST_MAX_CHANNELS)
    return fail(NEST_ERR_UNSUPPORTED, "in_features must be in [1, %d]", NEST_MAX_CHANNELS);
  const int dt = mlp->dtype;
  if (dt != NEST_DTYPE_F32 && dt != NEST_DTYPE_F16 && dt != NEST_DTYPE_BF16)
    return fail(NEST_ERR_UNSUPPORTED, "MLP dtype must be float32, float16 or bfloat16");
  if (dt == NEST_DTYPE_F32) {
    if (mlp->width != 16 && mlp->width != 32 && mlp->width != 64)
      return fail(NEST_ERR_UNSUPPORTED, "float32 MLP width must be 16, 32 or 64 (got %d)", mlp->width);
  } else {
    if (mlp->width != 32 && mlp->width != 64 && mlp->width != 128)
      return fail(NEST_ERR_UNSUPPORTED, "MFMA MLP width must be 32, 64 or 128 (got %d)", mlp->width);
    if (mlp->in_features % 16 != 0)
      return fail(NEST_ERR_UNSUPPORTED, "MFMA MLP needs in_features to be a multiple of 16 (got %d)", mlp->in_features);
  }
  if (!dirs && (!ray_matrix || width <= 0))
    return fail(NEST_ERR_INVALID_ARGUMENT, "either dirs or ray_matrix with the image width is required");
  if (N == 0) return NEST_OK;
  if (!feat || !out || !mlp->w1 || !mlp->w2 || !mlp->w3) return fail(NEST_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  MlpParams p{};
  p.C = mlp->in_features;
  p.width = mlp->width;
  p.dtype = dt;
  p.w1 = mlp->w1;
  p.w2 = mlp->w2;
  p.w3 = mlp->w3;
  p.feat = feat;
  p.feat_cs = feat_cs;
  p.feat_ns = feat_ns;
  p.N = N;
  p.img_w = width > 0 ? width : 1;
  p.dirs = dirs;
  if (ray_matrix) memcpy(p.M, ray_matrix, sizeof(p.M));
  p.alpha = alpha;
  if (bg) {
    memcpy(p.bg, bg, sizeof(p.bg));
    p.use_bg = (bg[0] + bg[1] + bg[2]) > 0.0f;
  }
  p.out = out;
  p.out_os = out_os;
  p.out_ns = out_ns;
  hipError_t e = launch_mlp(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "mlp_decode");
}

namespace {
// Validates one attribute's decode arguments and fills p (nothing to launch
// when P == 0).
int rvq_params(int64_t P, int32_t stages, int32_t K, int32_t dim, const float* cb, const uint16_t* idx,
               const float* bias, int32_t activation, float* out, float* raw_out, RvqParams& p) {
  if (P < 0) return fail(NEST_ERR_INVALID_ARGUMENT, "P must be >= 0");
  if (stages < 1 || stages > 16) return fail(NEST_ERR_UNSUPPORTED, "stages must be in [1, 16]");
  if (K < 1 || K > 65536) return fail(NEST_ERR_UNSUPPORTED, "codebook size must be in [1, 65536]");
  if (dim != 1 && dim != 2 && dim != 3 && dim != 4 && dim != 8)
    return fail(NEST_ERR_UNSUPPORTED, "dim must be 1, 2, 3, 4 or 8 (got %d)", dim);
  if (activation < 0 || activation > 3) return fail(NEST_ERR_INVALID_ARGUMENT, "activation must be 0..3");
  if (P > 0 && (!cb || !idx || !out)) return fail(NEST_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  p = RvqParams{};
  p.P = P;
  p.stages = stages;
  p.K = K;
  p.dim = dim;
  p.cb = cb;
  p.idx = idx;
  if (bias) {
    for (int d = 0; d < dim; d++) p.bias[d] = bias[d];
    p.has_bias = 1;
  }
  p.activation = activation;
  p.out = out;
  p.raw = raw_out;
  return NEST_OK;
}
}  // namespace

int nest_rvq_decode(int64_t P, int32_t stages, int32_t K, int32_t dim, const float* cb, const uint16_t* idx,
                    const float* bias, int32_t activation, float* out, float* raw_out, void* stream) {
  RvqParams p{};
  const int rc = rvq_params(P, stages, K, dim, cb, idx, bias, activation, out, raw_out, p);
  if (rc || P == 0) return rc;
  hipError_t e = launch_rvq(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "rvq_decode");
}

int nest_rvq_decode_batch(int32_t n, const nest_rvq_attr* attrs, void* stream) {
  if (n < 0 || n > NEST_RVQ_BATCH_MAX)
    return fail(NEST_ERR_INVALID_ARGUMENT, "n must be in [0, %d] (got %d)", NEST_RVQ_BATCH_MAX, n);
  if (n > 0 && !attrs) return fail(NEST_ERR_INVALID_ARGUMENT, "attrs is NULL");
  RvqBatch b{};
  for (int k = 0; k < n; k++) {
    const nest_rvq_attr& a = attrs[k];
    if (a.struct_size != sizeof(nest_rvq_attr))
      return fail(NEST_ERR_INVALID_ARGUMENT, "nest_rvq_attr[%d].struct_size mismatch", k);
    const int rc = rvq_params(a.P, a.stages, a.codebook_size, a.dim, a.codebooks, a.indices, a.bias, a.activation,
                              a.out, a.raw_out, b.a[b.n]);
    if (rc) return rc;
    if (a.P > 0) b.n++;
  }
  hipError_t e = launch_rvq_batch(b, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NEST_OK : hip_fail(e, "rvq_decode_batch");
}

}  // extern "C"
