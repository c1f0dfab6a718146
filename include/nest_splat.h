/*
 * nest_splat.h -- C ABI of the MI355X (gfx950) forward renderer for neural
 * shell texture splatting: 2D-surfel preprocess, tile binning with a radix
 * sort, per-tile compositing with an in-loop multi-level hash-grid lookup,
 * view-direction MLP decode on MFMA, RVQ attribute decode.
 *
 * Conventions
 *  - Every pointer named "device" is HIP device memory owned by the caller;
 *    the library never allocates device memory.  Scratch comes in through
 *    caller-provided workspaces whose sizes the *_workspace_size / *_layout
 *    queries report; the one exception is nest_inclusive_scan_u32_noalloc,
 *    whose scratch is a fixed 512 KiB device array the library owns.
 *  - Every launch is ordered on the caller's stream (a hipStream_t passed as
 *    void*, NULL = the null stream).  The only host synchronisation is the
 *    read-back of the number of tile/splat pairs in nest_forward_geometry
 *    (the reference reads it the same way, rasterizer_impl.cu:359).
 *  - Every entry point returns NEST_OK (0) or a negative status.  Arguments
 *    are validated before the first launch, so an error return leaves every
 *    output untouched.  nest_last_error() gives the message of the last failed
 *    call on the calling thread.
 *  - Reference citations are relative to the NilKel/nest-splatting tree:
 *      CR/  = submodules/diff-surfel-rasterization/cuda_rasterizer/
 *      DSR/ = submodules/diff-surfel-rasterization/
 *      GE/  = gridencoder/,  HE = hash_encoder/modules.py
 */
#ifndef NEST_SPLAT_H
#define NEST_SPLAT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NEST_ABI_VERSION 17

#define NEST_OK 0
#define NEST_ERR_INVALID_ARGUMENT (-1)
#define NEST_ERR_UNSUPPORTED (-2)
#define NEST_ERR_WORKSPACE (-3)
#define NEST_ERR_HIP (-4)
#define NEST_ERR_OVERFLOW (-5)

#define NEST_DTYPE_F32 0
#define NEST_DTYPE_F16 1
#define NEST_DTYPE_BF16 2

#define NEST_MAX_LEVELS 32
#define NEST_MAX_CHANNELS 128
#define NEST_OTHERS_CHANNELS 14 /* allmap channels, CR/auxiliary.h:24-31 */

/* Per-frame rasterizer settings: GaussianRasterizationSettings
 * (DSR/diff_surfel_rasterization/__init__.py:277-293).  Matrices are the
 * reference's flat float[16] world_view_transform / full_proj_transform. */
typedef struct nest_raster_settings {
  uint32_t struct_size;
  int32_t image_height;
  int32_t image_width;
  float tanfovx;
  float tanfovy;
  float scale_modifier;
  float viewmatrix[16];
  float projmatrix[16];
  float campos[3];
  float beta;
  int32_t prefiltered;
  int32_t debug;              /* synchronise and check after every stage */
  int32_t if_contract;
  uint32_t max_intersections; /* 0 = unlimited */
} nest_raster_settings;

/* Hash grid seen by the render loop: HashGridSettings (DSRpy:295-302) plus the
 * GridEncoder parameters of GE/grid.py:164-165.  offsets and gridrange are
 * host copies of the reference's device tensors. */
typedef struct nest_hashgrid {
  uint32_t struct_size;
  uint32_t levels;            /* L queried; 0 selects the colours_precomp path in mode 0 */
  uint32_t level_dim;         /* F: 1, 2, 4 or 8 (3 in render modes 8-10, 12 in mode 1,
                                 15 in mode 5) */
  float log2_scale;           /* S = log2(per_level_scale) */
  uint32_t base_resolution;   /* H */
  int32_t align_corners;
  int32_t interpolation;      /* 0 linear, 1 smoothstep */
  int32_t table_dtype;        /* NEST_DTYPE_F32 or NEST_DTYPE_F16 */
  const void *table;          /* device, [table_rows, F] */
  int64_t table_rows;         /* rows of the table; must be >= offsets[levels] */
  int32_t offsets[NEST_MAX_LEVELS + 1];
  float gridrange[2];
  /* Feature composition of the render loop, the reference's render_mode
   * argument (DSRpy:393, CR/forward.cu:1127) with its packed level argument
   * decoded by the caller (GR:217-242, :334-405):
   *   NEST_MODE_BASELINE (0): the grid's `levels` levels, or the colour path
   *     when levels == 0;
   *   NEST_MODE_CAT (4): hybrid_levels*level_dim per-splat features
   *     (colors_precomp rows of that width), then the grid's `levels` levels
   *     (CR/forward.cu:1218-1282; the reference counts those levels from the
   *     offsets);
   *   NEST_MODE_ADAPTIVE_CAT_FAST (13), | NEST_MODE_INFERENCE for inference:
   *     colors_precomp rows of total_levels*level_dim features plus a blend
   *     weight; the first hybrid_levels*level_dim channels come from the row,
   *     the next `levels` levels from the grid, blended with the row in
   *     training; in inference a splat with weight > 0.5 takes its row
   *     without a grid lookup (CR/forward.cu:965-1101);
   *   NEST_MODE_ADAPTIVE_ADD (7): colors_precomp rows of
   *     total_levels*level_dim features plus a weight; every channel is
   *     weight * row + (1 - weight) * grid, the grid's `levels` levels then
   *     zero (hybrid_levels must be 0; CR/forward.cu:1326-1376); the
   *     backward writes the weight's gradient times weight * (1 - weight);
   *   NEST_MODE_ADAPTIVE (6): colors_precomp rows of out_color's channel
   *     count; the first levels*level_dim channels are 0.5 * row + 0.5 * grid
   *     at the hit, the rest 0 (CR/forward.cu:1283-1325); forward only (the
   *     reference's backward reads another row layout, CR/backward.cu:1041);
   *   NEST_MODE_ADAPTIVE_CAT (12), | NEST_MODE_INFERENCE for inference: the
   *     same rows and levels; the first hybrid_levels*level_dim channels take
   *     the row unweighted, the grid levels are blended with the row in
   *     training; in inference a splat with weight >= 0.9 takes its row
   *     without a grid lookup; every hit records its world position,
   *     appearance colour and last contributor (CR/forward.cu:1593-1713);
   *   NEST_MODE_ADAPTIVE_ZERO (14), | NEST_MODE_INFERENCE for inference:
   *     colors_precomp rows of hybrid_levels*level_dim features plus a
   *     weight; the grid's `levels` levels follow, times the weight, when the
   *     weight is > 1e-6 (training) or >= 0.1 (inference), else zero; full
   *     hits (CR/forward.cu:1716-1830);
   *   NEST_MODE_HYBRID_SH (8), NEST_MODE_HYBRID_SH_POST (9),
   *   NEST_MODE_HYBRID_SH_RAW (10) (CR/forward.cu:1378-1542; GR:605-680):
   *     a grid of at most one level with level_dim 3 (float32) looked up at
   *     the hit, and colors_precomp rows of 3 raw SH colours (8, 10) or of 48
   *     SH coefficients channel-major (9; DC terms at 0, 16, 32).  Mode 8
   *     writes clamp(clamp(raw + 0.5, 0, 1) + sigmoid(grid), 0, 1), mode 10
   *     sigmoid(raw + grid), mode 9 the coefficients with the grid added to
   *     the DC terms; `decompose` 1 (gaussian_only) leaves the grid out, 2
   *     (ngp_only) the colour.  out_color needs 3 (8, 10) or 48 (9)
   *     channels; the channels past them stay 0.
   *   NEST_MODE_BASELINE_DOUBLE (2), NEST_MODE_BASELINE_BLEND_DOUBLE (3)
   *     (CR/forward.cu:1146-1217, :1975-2004): a second grid (table2,
   *     offsets2, gridrange2; the first grid's scale, base resolution and
   *     flags) queried at each splat's centre into rows2; mode 2 writes the
   *     first grid's `levels` levels at the hit, then those centre features;
   *     mode 3 blends only the centre features, then adds the first grid at
   *     the pixel's blended position with the appearance level of its tile's
   *     first splat.  level_dim 4; at most 64 channels (levels <= 8 in mode 2,
   *     16 in mode 3); table2 NULL leaves the centre features 0;
   *   NEST_MODE_SURFACE (1), NEST_MODE_SURFACE_RGB (5) (CR/forward.cu:
   *     1825-1908): float32 grid levels of 12 (mode 1) or 15 (mode 5)
   *     features at the hit, whose first 12 are four 3-vectors dotted with
   *     the splat's normal; mode 1 writes max(0, -dot + b) per vector, b the
   *     second grid's 4 features per level at the splat centre (0 without
   *     table2), 4 channels per level (levels <= 16); mode 5 max(0, -dot) and
   *     then the grid's features 12-14 at the centre, 7 channels per level
   *     (levels <= 9).  rows2 as in modes 2 and 3.
   * Modes 4, 7 and 12-14 need level_dim 2, 4 or 8 and at most 64 channels of
   * per-splat plus grid features; `levels` may be 0 there. */
  int32_t render_mode;
  uint32_t hybrid_levels;
  uint32_t total_levels;
  /* Render mode 4, backward only: the active grid-level count of the
   * reference's packed level (bits 8-15, coarse-to-fine training).  The
   * reference's backward copies the offsets only up to it and differentiates
   * the grid levels up to the last one whose offsets increase within that
   * copy (CR/backward.cu:576-612, :993-999), while the forward renders all
   * `levels`; nest_backward does the same.  The forward ignores it. */
  uint32_t active_levels;
  /* Render modes 8-10: 0 both parts, 1 gaussian_only, 2 ngp_only (bits 24-31
   * of the reference's packed level, GR:619-626).  Other modes ignore it. */
  uint32_t decompose;
  /* Render modes 1, 2 and 3: the second ("diffuse") grid, float32
   * [table2_rows, 4] with its own offsets and range (GR's features_diffuse,
   * offsets_diffuse, gridrange_diffuse), or table2 NULL; rows2 is the
   * caller's device scratch of [P, levels * 4] floats that the forward fills
   * with its features at the splat centres.  Other modes ignore them. */
  const void *table2;
  int64_t table2_rows;
  int32_t offsets2[NEST_MAX_LEVELS + 1];
  float gridrange2[2];
  float *rows2;
} nest_hashgrid;

#define NEST_MODE_BASELINE 0
#define NEST_MODE_SURFACE 1
#define NEST_MODE_BASELINE_DOUBLE 2
#define NEST_MODE_BASELINE_BLEND_DOUBLE 3
#define NEST_MODE_SURFACE_RGB 5
#define NEST_MODE_ADAPTIVE 6
#define NEST_MODE_CAT 4
#define NEST_MODE_ADAPTIVE_ADD 7
#define NEST_MODE_HYBRID_SH 8
#define NEST_MODE_HYBRID_SH_POST 9
#define NEST_MODE_HYBRID_SH_RAW 10
#define NEST_MODE_ADAPTIVE_CAT 12
#define NEST_MODE_ADAPTIVE_CAT_FAST 13
#define NEST_MODE_ADAPTIVE_ZERO 14
#define NEST_MODE_INFERENCE 0x100

/* Splat attributes (device, float32, contiguous), as the reference passes them
 * to _C.rasterize_gaussians (DSRpy:105-146). */
typedef struct nest_splats {
  uint32_t struct_size;
  int32_t P;
  const float *means3D;        /* [P,3] */
  const float *scales;         /* [P,2] activated */
  const float *rotations;      /* [P,4] (w,x,y,z) */
  const float *opacities;      /* [P,1] activated */
  const float *homotrans;      /* [P,4,4] build_H, hash path */
  const float *ap_level;       /* [P,1] appearance level, NULL = no cap */
  const float *colors_precomp; /* [P,channels], colour path (levels == 0) */
  const float *shs;            /* [P,sh_coeffs,3] SH coefficients: colour path with
                                  3 channels when colors_precomp is NULL
                                  (computeColorFromSH, CR/forward.cu:21-72) */
  int32_t sh_degree;           /* active SH degree, 0..3 */
  int32_t sh_coeffs;           /* coefficients per splat, >= (sh_degree+1)^2 */
  /* kernel_type (CR/forward.cu:864-921, CR/backward.cu:764-812): 0 Gaussian
   * (the global beta activation of the settings), 1 beta kernel
   * opacity * (1 - rho)^shape with rho < 1, 2 flex (the Gaussian with a per-splat
   * beta activation), 3 general exp(-0.5 * max(rho, 1e-8)^(shape / 2)); the
   * per-splat parameter is shapes[i] (f32 [P], required for 1-3). */
  const float *shapes;
  int32_t kernel_type;
  int32_t reserved;
} nest_splats;

/* Frame outputs (device): out_color [channels,H,W], out_others [14,H,W] and
 * radii [P], the tensors RasterizeGaussiansCUDA returns
 * (DSR/rasterize_points.cu:156-166, :241). */
typedef struct nest_frame_outputs {
  uint32_t struct_size;
  int32_t channels;
  float *out_color;
  float *out_others;
  int32_t *radii;
  /* record_transmittance (DSR/rasterize_points.cu:169-171, CR/forward.cu:1961-1964):
   * NULL for both = off.  Otherwise f32 [P] each, zeroed by nest_forward_render,
   * then every hit that reaches the blend (every render mode but 13, whose
   * hits leave the loop first) adds 1 to cover_pixels[splat] and the pixel's
   * transmittance before the hit to trans_avg[splat] (a sum, as in the
   * reference; the reference's [P, 1] tensors). */
  float *cover_pixels;
  float *trans_avg;
} nest_frame_outputs;

/* Optional per-stage device times.  When enabled, the forward calls record a
 * pair of HIP events around each stage on the caller's stream (no extra
 * synchronisation); nest_timing_read() waits for the last recorded event and
 * fills ms[].  The events are created on first use and owned by the struct
 * until nest_timing_release(). */
#define NEST_STAGE_PREPROCESS 0
#define NEST_STAGE_SCAN 1
#define NEST_STAGE_DUPLICATE 2
#define NEST_STAGE_SORT 3
#define NEST_STAGE_RANGES 4
#define NEST_STAGE_RENDER 5
#define NEST_STAGE_DEPTH_ORDER 6   /* the splats' depth order, queued by nest_forward_geometry */
#define NEST_STAGE_COUNT 7
typedef struct nest_timing {
  uint32_t struct_size;
  int32_t enabled;
  float ms[NEST_STAGE_COUNT];
  void *events[2 * NEST_STAGE_COUNT]; /* library-owned hipEvent_t handles */
  uint32_t recorded;                  /* bit s set: stage s was recorded */
} nest_timing;
int nest_timing_read(nest_timing *timing);
int nest_timing_release(nest_timing *timing);

/* ---- library ---------------------------------------------------------- */

int nest_abi_version(void);
const char *nest_last_error(void);

/* ---- workspaces: GeometryState / BinningState / ImageState --------------
 * Replace the byte-buffer carving of CR/rasterizer_impl.cu:212-250 and
 * CR/rasterizer_impl.h:21-73.  Layout queries give the byte offset of each
 * array so callers (and tests) can read intermediate results. */
#define NEST_GEOM_DEPTH 0          /* f32 [P]                         */
#define NEST_GEOM_XY 1             /* f32 [P,2]                       */
#define NEST_GEOM_TILES 2          /* u32 [P]    tiles touched        */
#define NEST_GEOM_OFFSETS 3        /* u32 [P]    inclusive scan       */
#define NEST_GEOM_RECORDS 4        /* f32 [P,32] packed render record:
                                      0-2 Tu, 3-5 Tv, 6-8 Tw, 9-10 xy,
                                      11 opacity, 12-14 view normal,
                                      15 floor(ap_level) as uint32 bits,
                                      16-18 / 19-21 / 22-24 homotrans
                                      columns 0 / 1 / 3, 25 rho cut,
                                      27 depth, 28-31 acceptance bbox
                                      (x0, x1, y0, y1)                 */
#define NEST_GEOM_RADII 5          /* i32 [P]                         */
#define NEST_GEOM_SCAN_TMP 6       /* scan scratch                    */
#define NEST_GEOM_DEPTH_ORDER 7    /* u32 [P]    splat ids by (depth bits, id),
                                      culled splats last (queued by
                                      nest_forward_geometry)           */
#define NEST_GEOM_ORDER_OFFSETS 8  /* u32 [P]    exclusive scan of tiles
                                      touched in that order            */
#define NEST_GEOM_ORDER_TMP 9      /* depth sort scratch              */
#define NEST_GEOM_RGB 10           /* f32 [P,3]  colour from SH (when shs is set) */
#define NEST_GEOM_CLAMPED 11       /* u8  [P,3]  SH colour channel clamped to 0 */
#define NEST_GEOM_RECT 12          /* u32 [P,2]  tile rectangle [x0, x1) x
                                      [y0, y1) as (x0 | y0 << 16,
                                      x1 | y1 << 16), zeros when culled */
#define NEST_GEOM_ORDER_RECT 13    /* u32 [P,2]  the rectangles in depth order */
#define NEST_GEOM_FIELDS 14
int nest_geom_layout(int32_t P, size_t offsets[NEST_GEOM_FIELDS], size_t *total_bytes);

/* The pairs are emitted in depth order and sorted on the tile bits only;
 * VALS equals the reference's point_list.  nest_forward_render leaves KEYS
 * unwritten (nothing downstream reads them); nest_binning_keys fills it with
 * the reference's point_list_keys. */
#define NEST_BIN_PAIR_TILES 0      /* u32 [NR] tile id of each pair, pairs in depth order */
#define NEST_BIN_PAIR_IDS 1        /* u32 [NR] splat id of each pair, same order          */
#define NEST_BIN_KEYS 2            /* u64 [NR] sorted (tile << 32 | depth bits) */
#define NEST_BIN_VALS 3            /* u32 [NR] sorted (point_list) */
#define NEST_BIN_SORT_TMP 4
#define NEST_BIN_FIELDS 5
int nest_binning_layout(int64_t num_rendered, size_t offsets[NEST_BIN_FIELDS], size_t *total_bytes);

#define NEST_IMG_RANGES 0          /* u32 [tiles,2] */
#define NEST_IMG_FINAL_T 1         /* f32 [3,H,W]  (T, M1, M2)   */
#define NEST_IMG_N_CONTRIB 2       /* u32 [2,H,W]  (last, median) */
#define NEST_IMG_LEVELS 3          /* 16 B [NEST_MAX_LEVELS] per-level lookup constants
                                      of the hash grid, written by nest_forward_render */
#define NEST_IMG_TILE_ORDER 4      /* u32 [tiles]  render launch order: tiles by descending
                                      pair count (bucketed), written by nest_forward_render */
#define NEST_IMG_FIELDS 5
int nest_image_layout(int32_t width, int32_t height, size_t offsets[NEST_IMG_FIELDS], size_t *total_bytes);

/* Per-level constants of the hash grid as the lookups use them, for the
 * grid's `levels` levels: scale = exp2(l * S) * H - 1 (float), resolution =
 * ceil(scale) + 1, hashed = 1 when the level indexes by fast_hash (the
 * stride loop of get_grid_index exceeds the level's size), else 0 (dense);
 * query_feature, CR/hashgrid.h:122-124 and :7-40.  Host-only (no device
 * access); any output pointer may be NULL. */
int nest_hashgrid_levels(const nest_hashgrid *grid, float *scale, uint32_t *resolution, uint32_t *hashed);

/* ---- forward rasterizer -------------------------------------------------
 * Together these two calls are RasterizeGaussiansCUDA
 * (DSR/rasterize_points.cu:40-242) / CudaRasterizer::Rasterizer::forward
 * (CR/rasterizer_impl.cu:255-440) for render_mode 0, 4 and 13, split at the
 * num_rendered read-back (CR/rasterizer_impl.cu:359) so that the caller can
 * size the binning workspace in between, as the resize callbacks
 * (DSR/rasterize_points.cu:31-37) do in the reference.
 *
 * nest_forward_geometry: preprocessCUDA (CR/forward.cu:323-441) plus the
 * inclusive scan of tiles touched (CR/rasterizer_impl.cu:355); writes radii
 * and the total number of tile/splat pairs (waiting for that read-back only).
 * It also queues the splats' depth order, which does not depend on the pair
 * count, behind the read-back, so the GPU runs it while the caller sizes the
 * binning workspace; nest_forward_render reads it from the geometry
 * workspace. */
int nest_forward_geometry(const nest_raster_settings *settings, const nest_splats *splats,
                          void *geom_ws, size_t geom_bytes, int32_t *radii,
                          int64_t *num_rendered, nest_timing *timing, void *stream);

/* nest_forward_render: duplicateWithKeys (CR/rasterizer_impl.cu:70-111),
 * the radix sort on (tile|depth) keys (:378-386), identifyTileRanges
 * (:173-195, :388) and renderCUDAsurfelForward<C, render_mode>
 * (CR/forward.cu:639-2049, dispatch :2052-2158).  out_color channels must
 * cover the features of the mode (levels*level_dim in mode 0, plus
 * hybrid_levels*level_dim in mode 4, total_levels*level_dim in modes 7, 12-14);
 * channels past them are written as zero. */
int nest_forward_render(const nest_raster_settings *settings, const nest_hashgrid *grid,
                        const nest_splats *splats, void *geom_ws, size_t geom_bytes,
                        void *binning_ws, size_t binning_bytes, void *image_ws, size_t image_bytes,
                        int64_t num_rendered, const nest_frame_outputs *out,
                        nest_timing *timing, void *stream);

/* The reference's sorted keys point_list_keys, tile << 32 | depth bits of the
 * pair's splat (CR/rasterizer_impl.cu:381-386, binningState), written into the
 * binning workspace's NEST_BIN_KEYS slot from the tile ranges, the sorted point
 * list and the depths in the workspaces of a nest_forward_render call with the
 * same image size, P and num_rendered.  The reference has no separate call:
 * its sort writes them, while nest_forward_render sorts without them because
 * nothing downstream reads them (the backward walks ranges and point_list). */
int nest_binning_keys(int32_t width, int32_t height, int32_t P, const void *geom_ws, size_t geom_bytes,
                      void *binning_ws, size_t binning_bytes, const void *image_ws, size_t image_bytes,
                      int64_t num_rendered, void *stream);

/* ---- backward (training) ------------------------------------------------
 * nest_backward is RasterizeGaussiansBackwardCUDA
 * (DSR/rasterize_points.cu:243-471) / CudaRasterizer::Rasterizer::backward
 * (CR/rasterizer_impl.cu:444-600) for render modes 0, 4 and 12 (mode 4:
 * CR/backward.cu:987-1040, gradients of the per-splat rows into dL_dcolors
 * [P, hybrid_levels*level_dim], of the grid's active levels into
 * dL_dfeatures; mode 12 in training, CR/backward.cu:1425-1520, gradients of
 * the rows and their blend weight into dL_dcolors [P, total_levels*level_dim
 * + 1], likewise mode 7, CR/backward.cu:1108-1189; mode 14 in training,
 * CR/backward.cu:1521-1590, into dL_dcolors
 * [P, hybrid_levels*level_dim + 1]) with the Gaussian kernel:
 * renderCUDAsurfelBackward
 * (CR/backward.cu:445-2049) then
 * preprocessCUDA backward (CR/backward.cu:2216-2274).  It reads the
 * workspaces of the nest_forward_geometry / nest_forward_render calls of the
 * same frame (unchanged since) and the same settings, grid and splats.  Every
 * gradient output is overwritten.  Hash tables must be binary32; at most 64
 * output channels.  dL_dmeans2D receives the reference's densification
 * statistic (dL/dTu.z * depth * W/2, dL/dTv.z * depth * H/2), not a
 * gradient.  Per-splat and table gradients are summed with float atomics, so
 * their low bits vary from run to run, as in the reference. */
#define NEST_BWD_DTRANSMAT 0       /* f32 [P,9]  dL/dT of the render            */
#define NEST_BWD_DHOMO 1           /* f32 [P,9]  dL/dhomotrans (columns 0, 1, 3) */
#define NEST_BWD_DNORMAL 2         /* f32 [P,3]  dL/dnormal (view space)        */
#define NEST_BWD_DCOLORS 3         /* f32 [P,C]  colour gradient when io->dL_dcolors is NULL */
#define NEST_BWD_GRADSUM 4         /* f32 [P]    |dL/dfeature| sum when io->dL_dgradsum is NULL */
#define NEST_BWD_FIELDS 5
int nest_backward_layout(int32_t P, int32_t channels, size_t offsets[NEST_BWD_FIELDS], size_t *total_bytes);

typedef struct {
    uint32_t struct_size;            /* sizeof(nest_backward_io) */
    int32_t channels;                /* C of the forward's out_color */
    const float *dL_dout_color;      /* [C,H,W] */
    const float *dL_dout_others;     /* [14,H,W]; channels 0-6 carry gradient */
    float *dL_dmeans3D;              /* [P,3] */
    float *dL_dmeans2D;              /* [P,3] densification statistic */
    float *dL_dcolors;               /* [P,C] colour path, [P,hybrid_levels*level_dim]
                                        in render mode 4, [P,total_levels*level_dim+1]
                                        in render mode 12, [P,hybrid_levels*level_dim+1]
                                        in render mode 14, or NULL */
    float *dL_dopacity;              /* [P] */
    float *dL_dshs;                  /* [P,sh_coeffs,3] when the colours came from SH */
    float *dL_dscales;               /* [P,2] */
    float *dL_drotations;            /* [P,4] */
    float *dL_dfeatures;             /* [table_rows, level_dim] hash path */
    float *dL_dgradsum;              /* [P] hash path (returned for ap_level), or NULL */
    float *dL_dshapes;               /* [P] the splats' kernel parameter (kernel_type 1-3,
                                        required then; CR/backward.cu:1864-1909), or NULL */
} nest_backward_io;

int nest_backward(const nest_raster_settings *settings, const nest_hashgrid *grid, const nest_splats *splats,
                  const void *geom_ws, size_t geom_bytes, const void *binning_ws, size_t binning_bytes,
                  const void *image_ws, size_t image_bytes, int64_t num_rendered, const nest_backward_io *io,
                  void *bwd_ws, size_t bwd_bytes, void *stream);


/* GaussianModel.get_homotrans (scene/gaussian_model.py:312-317):
 * build_H(build_rotation(rotations), scales, means3D) of
 * utils/general_utils.py:78-113, the [P,4,4] row-major splat-to-world
 * transforms the forward reads (columns 0, 1 and 3).  rotations [P,4]
 * (w, x, y, z; normalised here as the reference does), scales [P,2],
 * means3D [P,3], homotrans [P,4,4]; device float32 arrays, rotations and
 * homotrans 16-byte aligned, scales 8-byte aligned.  Bit-exact with the
 * reference's float32 expressions. */
int nest_build_homotrans(int64_t P, const float *rotations, const float *scales, const float *means3D,
                         float *homotrans, void *stream);

/* markVisible (DSR/rasterize_points.cu:452-470, CR/rasterizer_impl.cu:198-210,
 * checkFrustum :54-66): present[i] = 1 when the view-space depth of
 * means3D[i] exceeds 0.2 (in_frustum, CR/auxiliary.h:190-215), else 0.
 * viewmatrix is the host copy of the 4x4 world-to-view matrix (the flat
 * float[16] the kernels read); present is a device byte array [P]. */
int nest_mark_visible(int32_t P, const float *means3D, const float viewmatrix[16], uint8_t *present,
                      void *stream);

/* ---- building blocks ----------------------------------------------------- */

/* cub::DeviceScan::InclusiveSum on uint32 (CR/rasterizer_impl.cu:223, :355). */
size_t nest_scan_workspace_size(int64_t n);
int nest_inclusive_scan_u32(const uint32_t *in, uint32_t *out, int64_t n, void *ws, size_t ws_bytes,
                            void *stream);

/* Allocation-free variant of nest_inclusive_scan_u32.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * block partials live in a 512 KiB device array owned by the library, one per
 * GPU, held until the process ends; n may be at most NEST_SCAN_NOALLOC_MAX
 * (larger n returns NEST_ERR_WORKSPACE before any launch).  The call
 * allocates nothing.  All calls on one GPU share that array, so calls that
 * overlap on one GPU (different streams or threads) race; calls ordered on
 * one stream do not.  Results equal nest_inclusive_scan_u32's. */
#define NEST_SCAN_NOALLOC_MAX 268431360 /* 65535 blocks of 4096 elements */
int nest_inclusive_scan_u32_noalloc(const uint32_t *in, uint32_t *out, int64_t n, void *stream);

/* cub::DeviceRadixSort::SortPairs, stable, on key bits [0, end_bit)
 * (CR/rasterizer_impl.cu:245-249, :381-386). */
size_t nest_sort_workspace_size(int64_t n);
int nest_sort_pairs_u64(const uint64_t *keys_in, const uint32_t *vals_in, uint64_t *keys_out,
                        uint32_t *vals_out, int64_t n, int32_t end_bit, void *ws, size_t ws_bytes,
                        void *stream);

/* GridEncoder forward: grid_encode_forward (GE/src/gridencoder.cu:450-473,
 * kernel_grid :87-242) for gridtype hash (0) or tiled (1).  inputs [B,D] in
 * [0,1], embeddings [emb_rows, C] of emb_dtype (F32 or F16) with
 * emb_rows >= offsets[L], offsets a host array of L+1 entries.  outputs
 * [B, L*C] of emb_dtype: the permuted layout GE/grid.py:59 returns, written
 * directly. */
int nest_grid_encode(const float *inputs, int64_t B, int32_t D, const void *embeddings,
                     int64_t emb_rows, int32_t emb_dtype, const int32_t *offsets_host, int32_t L, int32_t C, float S,
                     int32_t H, int32_t gridtype, int32_t align_corners, int32_t interpolation,
                     void *outputs, void *stream);

/* GridEncoder.backward (GE/grid.py:70-91, GE/src/gridencoder.cu:245-366):
 * grad_embeddings [emb_rows, C] is overwritten with the table gradient of
 * grad [B, L*C]; grad_inputs [B, D] (or NULL) receives the input gradient
 * through the forward's dy_dx (gridencoder.cu:196-242).  Arguments as
 * nest_grid_encode; D must be 3 and the embeddings binary32. */
int nest_grid_encode_backward(const float *inputs, int64_t B, int32_t D, const void *embeddings, int64_t emb_rows,
                              int32_t emb_dtype, const int32_t *offsets_host, int32_t L, int32_t C, float S, int32_t H,
                              int32_t gridtype, int32_t align_corners, int32_t interpolation, const float *grad,
                              float *grad_embeddings, float *grad_inputs, void *stream);

/* View-direction MLP decode: INGP.rgb_decode/get_color (HE:587-602) with the
 * SphericalHarmonics degree-4 view encoding of (d+1)/2 (HE:551-558, :727-730)
 * and a bias-free ReLU MLP in -> width -> width -> 3 with sigmoid output
 * (HE:560-572), fused with the mask and background composition of
 * gaussian_renderer/__init__.py:1013-1021.
 *  feat: float32, element (pixel n, channel c) at feat[c*feat_cstride + n*feat_nstride]
 *  dirs: unit view directions [N,3] float32, or NULL to derive them per pixel
 *        as (x, y, 1) @ ray_matrix (cam2rays, utils/point_utils.py:31-46,
 *        normalised) for N = height*width pixels in row-major order
 *  alpha: [N] or NULL; rgb = alpha > 0 ? rgb : 0, then + (1-alpha)*bg when
 *        bg[0]+bg[1]+bg[2] > 0
 *  weights: w1 [width, C+16], w2 [width, width], w3 [3, width] row-major in
 *        dtype (F16 and BF16 run on MFMA, F32 on the vector ALU)
 *  out: element (channel o, pixel n) at out[o*out_ostride + n*out_nstride] */
typedef struct nest_mlp {
  uint32_t struct_size;
  int32_t in_features;       /* C */
  int32_t width;             /* hidden width: 16..256, multiple of 16 */
  int32_t dtype;
  const void *w1;
  const void *w2;
  const void *w3;
} nest_mlp;
int nest_mlp_decode(const nest_mlp *mlp, const float *feat, int64_t feat_cstride, int64_t feat_nstride,
                    int64_t N, int32_t width, const float *dirs, const float ray_matrix[9],
                    const float *alpha, const float bg[3], float *out, int64_t out_ostride,
                    int64_t out_nstride, void *stream);

/* Residual-VQ attribute decode (no reference counterpart; defined by the
 * RVQ workload of the benchmark suite):
 *   raw[p][d] = bias[d] + (((cb[0][i0][d] + cb[1][i1][d]) + cb[2][i2][d]) + ...)
 * codebooks [stages, K, dim] float32, indices [P, stages] uint16, bias a host
 * array of dim floats or NULL.  activation: 0 none, 1 exp, 2 normalise
 * (v / max(|v|, 1e-12)), 3 sigmoid -- the GaussianModel activations
 * (scene/gaussian_model.py:26-41).  out [P,dim]; raw_out [P,dim] or NULL.
 * An index >= codebook_size is never dereferenced: that splat decodes to NaN. */
int nest_rvq_decode(int64_t P, int32_t stages, int32_t codebook_size, int32_t dim,
                    const float *codebooks, const uint16_t *indices, const float *bias,
                    int32_t activation, float *out, float *raw_out, void *stream);

/* Up to NEST_RVQ_BATCH_MAX attributes (e.g. scale, rotation, opacity) in one
 * launch, each with the arguments of nest_rvq_decode.  No counterpart in the
 * reference either; results equal separate nest_rvq_decode calls. */
#define NEST_RVQ_BATCH_MAX 4
typedef struct nest_rvq_attr {
  uint32_t struct_size;
  int64_t P;
  int32_t stages;
  int32_t codebook_size;
  int32_t dim;
  int32_t activation;
  const float *codebooks;
  const uint16_t *indices;
  const float *bias;    /* dim floats or NULL */
  float *out;
  float *raw_out;       /* or NULL */
} nest_rvq_attr;
int nest_rvq_decode_batch(int32_t n, const nest_rvq_attr *attrs, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NEST_SPLAT_H */
