// Launch parameters shared between the C ABI (abi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/nest_splat.h"

namespace nest {

constexpr int kTile = 16;               // 16x16 pixel tiles (CR/config.h:17-18)
constexpr int kRecordFloats = 32;       // packed per-splat render record, 128 B

// Packed render record (float index within the 32-float record):
//   0..2 Tu   3..5 Tv   6..8 Tw   9..10 xy   11 opacity
//  12..14 normal   15 appearance level (uint32 bits, floor(ap_level))
//  16..18 SuTu (homotrans col 0)   19..21 SvTv (col 1)   22..24 pk (col 3)
//  25 rho cut (alpha < 1/255 beyond it)   26 splat id (set when staged)
//  27 depth   28..31 acceptance bbox x0, x1, y0, y1 (pixels)
enum RecordField {
  kRecTu = 0, kRecTv = 3, kRecTw = 6, kRecXY = 9, kRecOpacity = 11,
  kRecNormal = 12, kRecAp = 15, kRecSu = 16, kRecSv = 19, kRecPk = 22, kRecCut = 25, kRecId = 26,
  kRecDepth = 27, kRecBBox = 28
};

struct PreprocessParams {
  int P;
  int W, H;
  uint32_t gx, gy;
  float scale_mod;
  float beta;               // render's G -> (1+beta) G / (1+beta G) activation (0: off)
  float view[16];
  float proj[16];
  const float* means;
  const float* scales;
  const float* rots;
  const float* opac;
  const float* homotrans;   // may be null (colour path)
  const float* ap_level;    // may be null
  const float* shs;         // [P, sh_coeffs, 3] or null: RGB from SH for the colour path
  int sh_degree;
  int sh_coeffs;
  float campos[3];
  int kernel_type;          // 0 Gaussian, 1 beta, 2 flex, 3 general
  const float* shapes;      // [P] per-splat kernel parameter (kernel_type 1-3), copied to record[26]
  // outputs
  int32_t* radii;
  int32_t* radii_user;      // optional second copy (the caller's radii tensor)
  float* xy;
  float* depth;
  uint32_t* tiles;
  uint32_t* rect;           // [P, 2] tile rectangle (x0 | y0 << 16, x1 | y1 << 16), zeros when culled
  uint32_t* depth_key;      // [P] key of the depth order: depth bits, 0xffffffff when culled
  float* records;
  float* rgb;               // [P, 3], written when shs is set
  uint8_t* clamped;         // [P, 3], written when shs is set
};

// markVisible: present[i] = 1 when splat i lies beyond the near plane.
hipError_t launch_mark_visible(int P, const float* means, const float view[16], uint8_t* present, hipStream_t s);
hipError_t launch_build_homotrans(int64_t P, const float* rots, const float* scales, const float* means, float* H,
                                  hipStream_t s);

// Per-level constants of the hash grid, computed on the host in the same
// float order as the reference's query_feature (CR/hashgrid.h:122-131).
struct LevelTable {
  float scale[NEST_MAX_LEVELS];
  uint32_t res1[NEST_MAX_LEVELS];      // resolution + 1 (or resolution if align_corners)
  uint32_t hsize[NEST_MAX_LEVELS];     // offsets[l+1] - offsets[l]
  uint32_t base[NEST_MAX_LEVELS];      // offsets[l] (entries, not floats)
  uint32_t flags[NEST_MAX_LEVELS];     // bit0 hashed, bit1 power-of-two size, bits 2.. stride count
};

// Per-level constants of the common-grid lookup (see GridParams::structured),
// one 16-byte record per level so that a level costs one scalar load:
// dense levels {scale, res1, res1^2, byte offset}, hashed levels
// {scale, size - 1, 0, byte offset}.
struct LevelQuad {
  float scale;
  uint32_t a;     // res1 (dense) or size - 1 (hashed, power of two)
  uint32_t b;     // res1 * res1 (dense) or 0 (hashed)
  uint32_t soff;  // first entry of the level, in bytes
};

struct GridParams {
  uint32_t L;           // levels queried
  uint32_t F;
  uint32_t interp;
  uint32_t contract;
  float vmin, vmax;
  float inv_size;       // 1/(vmax-vmin) or 1/((vmax-vmin)*0.5) in contract mode
  float vmid;
  float pos_offset;     // 0.5 or 0 (align_corners)
  uint32_t half;        // table entries are binary16
  uint32_t table_bytes; // byte size of the table (< 4 GiB: 32-bit buffer offsets)
  uint32_t table_rows;  // entries of the table (records of the struct-buffer view)
  uint32_t structured;  // levels [0, n_dense) dense without modulo, the rest hashed power-of-two
  uint32_t n_dense;
  LevelQuad* lq;        // [L] device copy of the level records (structured grids), written by launch_render
  const void* table;
  LevelTable lv;
};

struct RenderParams {
  int W, H;
  uint32_t gx, gy;
  uint32_t ntiles;
  int C;                 // out_color channels
  int level;             // 0 colour path, >0 hash
  float beta;
  uint32_t max_intersections;
  int kernel_type;            // 0 Gaussian, 1 beta, 2 flex, 3 general (shape in record[26])
  const uint32_t* ranges;     // [tiles][2]
  const uint32_t* point_list;
  const float* records;       // [P][32]
  const float* colors;        // [P][C] colour path; [P][cstride] per-splat features (mix)
  uint32_t* tile_order;       // [tiles] launch order, written by launch_render
  float* out_color;
  float* out_others;
  float* final_T;
  uint32_t* n_contrib;
  float* cover_pixels;        // record_transmittance: [P] hits per splat, or nullptr
  float* trans_avg;           // [P] sum of the transmittance before each hit
  GridParams grid;
  // Per-splat features ahead of the grid's (render modes 4, 12, 13, 14):
  // channel c < pgd of a hit is row[c] (times the row's weight with
  // wcoarse); grid level l lands on channels pgd + l*F.
  int mix;                    // 0: mode 0
  int hyb;                    // per-splat levels ahead of the grid's
  int pgd;                    // hyb * F
  int cstride;                // floats per row of colors
  int nrow;                   // leading floats of a row the render reads as features (<= 64)
  int wslot;                  // index of the blend weight in a row (modes 12, 13), else -1
  float wfix;                 // the blend weight without a weight slot (mode 6: 0.5)
  int infer;                  // inference: a fast hit (weight > 0.5 in mode 13, >= 0.9 in
                              // mode 12) takes the row without the grid
  int blend;                  // training: grid levels take row * weight + grid * (1 - weight)
  int m13;                    // mode 13: a hit updates no appearance colour and no last
                              // contributor, a fast hit adds no world position
  int wcoarse;                // mode 13 training: the first pgd channels take row * weight
  int gscale;                 // mode 14: grid levels take grid * weight
  float fthr;                 // a hit is fast (skips the grid) when (weight > fthr) != fneg;
  int fneg;                   // fthr = +inf: no fast hits
  uint32_t nfast;             // levels of the row past pgd that a fast hit takes
  uint32_t nblend;            // levels past pgd a blend hit covers: the grid's in modes 12, 13;
                              // the row's in mode 7 (the grid zero past its levels)
  // Hybrid SH modes 8, 9, 10 (0 otherwise): a hit's channels come from its
  // colors row (3 or 48 floats) and one 3-channel grid level at the hit;
  // hsh_dec 1 leaves the grid out, 2 the row's colour.  Surface-potential
  // modes 1 and 5: the grid's levels at the hit and the centre rows in colors.
  int hsh;
  int hsh_dec;
  // Render mode 2: the accumulators hold [centre rows | grid]; output channel
  // of accumulator c < rot_n is (c + rot) % rot_n, so the grid comes first.
  int rot;
  int rot_n;
};

// Host-side launchers (defined in the .hip files).  Each returns the
// hipGetLastError() of its launches.
hipError_t launch_preprocess(const PreprocessParams& p, hipStream_t s);
hipError_t launch_scan_u32(const uint32_t* in, uint32_t* out, int64_t n, void* ws, hipStream_t s);
size_t scan_ws_bytes(int64_t n);
size_t sort_ws_bytes(int64_t n);
// Stable sort of (keys_in, vals_in) on key bits [0, end_bit) into
// (keys_out, vals_out); the inputs are not written.
hipError_t launch_sort_pairs(const uint64_t* keys_in, const uint32_t* vals_in, uint64_t* keys_out, uint32_t* vals_out,
                             int64_t n, int end_bit, void* ws, hipStream_t s);
// Splat ids in (depth bits, id) order, culled splats last, their tile
// rectangles in that order and the exclusive scan of their tiles touched.
// ws starts with the P depth keys (PreprocessParams::depth_key).
size_t depth_order_ws_bytes(int P);
hipError_t launch_depth_order(int P, const uint32_t* rect, uint32_t* order, uint32_t* ordered_offsets,
                              uint32_t* ordered_rect, void* ws, hipStream_t s);
// (tile id, splat id) pairs of the splats in depth order, from their
// rectangles in that order; at most n_pairs are written.
hipError_t launch_duplicate_ordered(int P, const uint32_t* order, const uint32_t* offsets, const uint32_t* ordered_rect,
                                    uint32_t gx, int64_t n_pairs, uint32_t* tile_keys, uint32_t* ids, hipStream_t s);
// Stable sort of the depth-ordered pairs on tile bits [0, tile_bits): writes
// the splat ids in tile/depth order, the (tile << 32 | depth bits) keys too
// unless keys_out is NULL, and leaves the pairs per tile in ranges (ntiles
// uint2, count in .y, x zero) for launch_tile_ranges.
size_t tile_sort_ws_bytes(int64_t n);
hipError_t launch_sort_tiles(const uint32_t* tile_keys, const uint32_t* ids, uint64_t* keys_out, uint32_t* vals_out,
                             int64_t n, int tile_bits, const float* depth, uint32_t* ranges, uint32_t ntiles, void* ws,
                             hipStream_t s);
// Per-tile [start, end) of the n sorted pairs from those counts ((0, 0) for a
// tile without pairs); with n == 0, zeroes the ranges.
hipError_t launch_tile_ranges(uint32_t* ranges, int64_t n, uint32_t ntiles, hipStream_t s);
// point_list_keys (tile << 32 | depth bits) of the sorted pairs, from the tile
// ranges and the point list.
hipError_t launch_compose_keys(const uint32_t* ranges, const uint32_t* point_list, const float* depth, uint32_t ntiles,
                               uint64_t* keys, hipStream_t s);
hipError_t launch_render(const RenderParams& p, hipStream_t s);
// Render modes 2 and 3: the second grid g2 (4 features per level, float32)
// at every splat's centre (homotrans column 3), levels below min(ap, L), into
// rows [P, L * 4].
hipError_t launch_centre_rows(const GridParams& g2, int P, const float* homotrans, const float* ap_level, float* rows,
                              hipStream_t s);
// Render mode 5: the grid's (15 features per level, float32) features 12-14
// of each level at every splat's centre, into rows [P, L * 3].
hipError_t launch_centre_rgb(const GridParams& g, int P, const float* homotrans, const float* ap_level, float* rows,
                             hipStream_t s);
// Render mode 3 after the render: each pixel's out_color channels [0, L * 4)
// plus the grid p.grid at its blended position (out_others 8-10) with the
// appearance level of the tile's first splat (0 without hits or ap_level).
hipError_t launch_spatial_add(const RenderParams& p, const float* ap_level, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* dst, uint32_t value, int64_t n, hipStream_t s);

// Backward of the render (renderCUDAsurfelBackward, mode 0).  Reads the
// forward's records, point list, ranges, final_T and n_contrib; accumulates
// into zero-filled gradient arrays.
struct RenderBwdParams {
  int W, H;
  uint32_t gx, gy;
  uint32_t ntiles;
  int C;
  int level;                  // 0 colour path, >0 hash
  float beta;
  const uint32_t* ranges;
  const uint32_t* point_list;
  const uint32_t* tile_order; // [tiles] the forward's launch order (heaviest tiles first)
  const float* records;       // [P][32]
  const float* colors;        // [P][C] colour path, [P][pgd] mode-4 rows
  const float* final_T;       // [3][H][W]
  const uint32_t* n_contrib;  // [2][H][W]
  const float* dL_dpix;       // [C][H][W]
  const float* dL_dothers;    // [14][H][W]
  float* dtable;              // [rows][F] hash path
  float* dtransmat;           // [P][9]
  float* dhomo;               // [P][9]
  float* dmean2D;             // [P][3]
  float* dnormal;             // [P][3]
  float* dopacity;            // [P]
  float* dcolors;             // [P][C] colour path, [P][pgd] per-splat rows
  float* gradsum;             // [P] hash path
  int pgd;                    // render modes 4, 12: per-splat (coarse) channels of a row (0 otherwise)
  int cstride;                // render mode 12: floats per row (total*F + 1)
  int wslot;                  // render modes 12, 14: index of the blend weight in a row, else -1
  int azero;                  // render mode 14: grid levels take grid * weight, no row part
  int wsig;                   // render mode 7: the weight slot gets dL/dweight * w * (1 - w)
  int nfine;                  // render modes 12, 14: grid channels after the coarse ones (levels * F)
  int kernel_type;            // 0 Gaussian, 1 beta, 2 flex, 3 general (shape in record[26])
  float* dshapes;             // [P] kernel types 1-3
  GridParams grid;
};
hipError_t launch_render_backward(const RenderBwdParams& p, hipStream_t s);

// Backward of preprocess (preprocessCUDA backward with compute_transmat_aabb
// and computeColorFromSH), one lane per splat with radii > 0.
struct PreprocessBwdParams {
  int P, W, H;
  float view[16];
  float proj[16];
  float campos[3];
  const float* means;
  const float* scales;
  const float* rots;
  const int32_t* radii;
  const float* records;       // [P][32]: Tw.z (depth of the statistic)
  const float* shs;           // [P][sh_coeffs][3] or null
  int sh_degree, sh_coeffs;
  const uint8_t* clamped;     // [P][3]
  const float* dcolors;       // [P][3] when shs
  const float* dtransmat;     // [P][9]
  const float* dhomo;         // [P][9]
  const float* dnormal;       // [P][3]
  float* dmean2D;             // [P][3]: read, then overwritten with the statistic
  float* dmeans;              // [P][3]
  float* dscales;             // [P][2]
  float* drots;               // [P][4]
  float* dshs;                // [P][sh_coeffs][3] when shs
};
hipError_t launch_preprocess_backward(const PreprocessBwdParams& p, hipStream_t s);

// GridEncoder backward, D = 3, binary32 table: table gradient (accumulated
// into a zero-filled array) and, when grad_inputs is set, the input gradient.
struct GridEncodeBwdParams {
  const float* inputs;    // [B][3]
  int64_t B;
  int F;
  int L;
  int align_corners;
  int interp;
  const float* table;
  uint32_t table_rows;
  const float* grad;      // [B][L*F]
  float* grad_table;      // [rows][F]
  float* grad_inputs;     // [B][3] or null
  LevelTable lv;
};
hipError_t launch_grid_encode_backward(const GridEncodeBwdParams& p, hipStream_t s);

struct GridEncodeParams {
  const float* inputs;
  int64_t B;
  int D;
  int C;                // features per level
  int L;
  int gridtype;
  int align_corners;
  int interp;
  int half;
  const void* table;
  void* outputs;
  LevelTable lv;
};
hipError_t launch_grid_encode(const GridEncodeParams& p, hipStream_t s);

// GridEncoder forward on the common level layout (D = 3, binary32 table,
// trilinear, levels [0, n_dense) dense without modulo and the rest hashed
// into power-of-two sizes): the render's level records and lookup.
struct GridEncodeQuadParams {
  const float* inputs;   // [B][3]
  int64_t B;
  int F;
  int L;
  float pos_offset;      // 0.5, or 0 with align_corners
  const float* table;
  uint32_t table_rows;
  float* outputs;        // [B][L*F]
  LevelQuad lq[NEST_MAX_LEVELS];
};
hipError_t launch_grid_encode_quad(const GridEncodeQuadParams& p, hipStream_t s);

struct MlpParams {
  int C;
  int width;
  int dtype;
  const void* w1;
  const void* w2;
  const void* w3;
  const float* feat;
  int64_t feat_cs, feat_ns;
  int64_t N;
  int img_w;
  const float* dirs;
  float M[9];
  const float* alpha;
  float bg[3];
  int use_bg;
  float* out;
  int64_t out_os, out_ns;
};
hipError_t launch_mlp(const MlpParams& p, hipStream_t s);

struct RvqParams {
  int64_t P;
  int stages;
  int K;
  int dim;
  const float* cb;
  const uint16_t* idx;
  float bias[8];
  int has_bias;
  int activation;
  float* out;
  float* raw;
};
hipError_t launch_rvq(const RvqParams& p, hipStream_t s);
constexpr int kRvqBatchMax = 4;
struct RvqBatch {
  RvqParams a[kRvqBatchMax];
  int n;
};
hipError_t launch_rvq_batch(const RvqBatch& b, hipStream_t s);

}  // namespace nest
