// Multi-level hash-grid lookup shared by the render kernel and GridEncoder.
//
// Semantics: query_feature / get_grid_index / fast_hash / smoothstep of
// submodules/diff-surfel-rasterization/cuda_rasterizer/hashgrid.h:7-212 and
// kernel_grid of gridencoder/src/gridencoder.cu:87-242 (D = 3).  The per-level
// scale, resolution and dense/hashed decision are host-computed constants
// (LevelTable) evaluated with the reference's uint32 stride loop, so the
// device code below only does the per-corner arithmetic.
#pragma once

#include <hip/hip_fp16.h>

#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

constexpr uint32_t kLvHashed = 1u;   // (res1)^3 > hashmap size in the uint32 loop
constexpr uint32_t kLvPow2 = 2u;     // hashmap size is a power of two
constexpr uint32_t kLvNoMod = 4u;    // dense and the linear index cannot reach the size

// F consecutive table values of entry e, widened to float.
template <int F, bool kHalf>
__device__ __forceinline__ void load_entry(const void* table, size_t e, float v[F]) {
  if constexpr (!kHalf) {
    const float* t = static_cast<const float*>(table);
    if constexpr (F == 4) {
      const float4 a = reinterpret_cast<const float4*>(t)[e];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else if constexpr (F == 2) {
      const float2 a = reinterpret_cast<const float2*>(t)[e];
      v[0] = a.x; v[1] = a.y;
    } else if constexpr (F == 8) {
      const float4 a = reinterpret_cast<const float4*>(t)[2 * e];
      const float4 b = reinterpret_cast<const float4*>(t)[2 * e + 1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int f = 0; f < F; f++) v[f] = t[e * F + f];
    }
  } else {
    const __half* t = static_cast<const __half*>(table);
    if constexpr (F == 4) {
      const uint2 a = reinterpret_cast<const uint2*>(t)[e];
      v[0] = __half2float(__ushort_as_half((unsigned short)(a.x & 0xffffu)));
      v[1] = __half2float(__ushort_as_half((unsigned short)(a.x >> 16)));
      v[2] = __half2float(__ushort_as_half((unsigned short)(a.y & 0xffffu)));
      v[3] = __half2float(__ushort_as_half((unsigned short)(a.y >> 16)));
    } else if constexpr (F == 2) {
      const uint32_t a = reinterpret_cast<const uint32_t*>(t)[e];
      v[0] = __half2float(__ushort_as_half((unsigned short)(a & 0xffffu)));
      v[1] = __half2float(__ushort_as_half((unsigned short)(a >> 16)));
    } else {
#pragma unroll
      for (int f = 0; f < F; f++) v[f] = __half2float(t[e * F + f]);
    }
  }
}

// Struct-buffer view of the table: one record per entry (stride = entry
// bytes in descriptor dword1[29:16]), num_records = rows, so the buffer unit
// scales the entry index (idxen addressing) and range-checks it.  clang has
// no struct-buffer load builtins, so the LLVM intrinsics are bound by name.
typedef int nest_i32x4 __attribute__((ext_vector_type(4)));
typedef int nest_i32x2 __attribute__((ext_vector_type(2)));
typedef float nest_f32x4 __attribute__((ext_vector_type(4)));
typedef float nest_f32x2 __attribute__((ext_vector_type(2)));
__device__ nest_f32x4 nest_struct_load_v4f32(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.v4f32");
__device__ nest_f32x2 nest_struct_load_v2f32(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.v2f32");
__device__ float nest_struct_load_f32(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.f32");
__device__ nest_i32x4 nest_struct_load_v4i32(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.v4i32");
__device__ nest_i32x2 nest_struct_load_v2i32(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.v2i32");
__device__ int nest_struct_load_i32(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.i32");
__device__ short nest_struct_load_i16(nest_i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.i16");
__device__ nest_i32x4 nest_raw_load_v4i32(nest_i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");

template <int F, bool kHalf>
__device__ __forceinline__ nest_i32x4 table_rsrc_rows(const void* table, uint32_t rows) {
  constexpr int kStride = F * (kHalf ? 2 : 4);
  const uint64_t a = reinterpret_cast<uint64_t>(table);
  nest_i32x4 r;
  r.x = (int)(uint32_t)(a & 0xffffffffu);
  r.y = (int)((uint32_t)((a >> 32) & 0xffffu) | ((uint32_t)kStride << 16));
  r.z = (int)rows;
  r.w = 0x00020000;
  return r;
}

// Byte-addressed view of the same table (stride 0, num_records = bytes):
// 16-byte loads that start at any entry of an 8-byte-entry table.  The table
// is below 4 GiB (the host checks), so rows * entry bytes fits 32 bits.
template <int F, bool kHalf>
__device__ __forceinline__ nest_i32x4 table_rsrc_raw(nest_i32x4 rows_view) {
  constexpr uint32_t kStride = F * (kHalf ? 2u : 4u);
  nest_i32x4 r = rows_view;
  r.y = (int)((uint32_t)r.y & 0xffffu);
  r.z = (int)((uint32_t)r.z * kStride);
  return r;
}

__device__ __forceinline__ float lo_half(uint32_t x) { return __half2float(__ushort_as_half((unsigned short)(x & 0xffffu))); }
__device__ __forceinline__ float hi_half(uint32_t x) { return __half2float(__ushort_as_half((unsigned short)(x >> 16))); }

template <int F, bool kHalf>
__device__ __forceinline__ void struct_entry(nest_i32x4 r, uint32_t index, uint32_t soff, float v[F]) {
  const int vi = (int)index, so = (int)soff;
  if constexpr (!kHalf) {
    if constexpr (F == 4) {
      const nest_f32x4 a = nest_struct_load_v4f32(r, vi, 0, so, 0);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else if constexpr (F == 2) {
      const nest_f32x2 a = nest_struct_load_v2f32(r, vi, 0, so, 0);
      v[0] = a.x; v[1] = a.y;
    } else if constexpr (F == 1) {
      v[0] = nest_struct_load_f32(r, vi, 0, so, 0);
    } else {
#pragma unroll
      for (int q = 0; q < F / 4; q++) {
        const nest_f32x4 a = nest_struct_load_v4f32(r, vi, 16 * q, so, 0);
        v[4 * q + 0] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
      }
    }
  } else {
    if constexpr (F == 4) {
      const nest_i32x2 a = nest_struct_load_v2i32(r, vi, 0, so, 0);
      v[0] = lo_half((uint32_t)a.x); v[1] = hi_half((uint32_t)a.x);
      v[2] = lo_half((uint32_t)a.y); v[3] = hi_half((uint32_t)a.y);
    } else if constexpr (F == 2) {
      const uint32_t a = (uint32_t)nest_struct_load_i32(r, vi, 0, so, 0);
      v[0] = lo_half(a); v[1] = hi_half(a);
    } else if constexpr (F == 8) {
      const nest_i32x4 a = nest_struct_load_v4i32(r, vi, 0, so, 0);
      const uint32_t w[4] = {(uint32_t)a.x, (uint32_t)a.y, (uint32_t)a.z, (uint32_t)a.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        v[2 * q] = lo_half(w[q]);
        v[2 * q + 1] = hi_half(w[q]);
      }
    } else {
      v[0] = lo_half((uint32_t)(uint16_t)nest_struct_load_i16(r, vi, 0, so, 0));
    }
  }
}

// Level l of the hash grid at u in [0,1]^3 through a struct-buffer view, with
// the reference's corner order (bit 0 +x, bit 1 +y, bit 2 +z), weights
// w = ((1 * wx) * wy) * wz and fused accumulation out = fmaf(w, v, out) from
// +0.  The corner indices are strength-reduced: with q = g + b (b in {0,1}^3)
// the hash is (g0+b0) ^ (g1*P1 + b1*P1) ^ (g2*P2 + b2*P2) and the dense index
// (g0 + g1 r + g2 r^2) + (b0 + b1 r + b2 r^2), both exact in uint32
// arithmetic, so a level needs two integer multiplies instead of two per
// corner.  The entry index goes to the buffer unit unscaled.
struct LevelCorners {
  uint32_t idx[8];   // entry index of corner k (bit 0: +x, bit 1: +y, bit 2: +z)
  uint32_t soff;     // byte offset of the level in the table
  uint32_t dense;    // wave-uniform: a dense level without modulo, so idx[2m + 1] == idx[2m] + 1
  float wx[2], wy[2], wz[2];
};

// Cell of u at a level: g = (uint32)floor(x) with the saturating conversion,
// pos = x - (float)g, x = u * scale + pos_offset, then the corner weights.
__device__ __forceinline__ void cell_weights(float scale, float pos_offset, bool smooth, const float u[3], uint32_t g[3],
                                             LevelCorners& cn) {
  float pos[3];
#pragma unroll
  for (int d = 0; d < 3; d++) {
    const float x = u[d] * scale + pos_offset;
    g[d] = f2u_sat(x);
    pos[d] = x - (float)g[d];
    if (smooth) pos[d] = pos[d] * pos[d] * (3.0f - 2.0f * pos[d]);
  }
  cn.wx[0] = 1 - pos[0]; cn.wx[1] = pos[0];
  cn.wy[0] = 1 - pos[1]; cn.wy[1] = pos[1];
  cn.wz[0] = 1 - pos[2]; cn.wz[1] = pos[2];
}

__device__ __forceinline__ void hashed_corners(const uint32_t g[3], uint32_t idx[8]) {
  const uint32_t a[2] = {g[0], g[0] + 1u};
  const uint32_t b0 = g[1] * 2654435761u, c0 = g[2] * 805459861u;
  const uint32_t b[2] = {b0, b0 + 2654435761u}, c[2] = {c0, c0 + 805459861u};
  const uint32_t ab[4] = {a[0] ^ b[0], a[1] ^ b[0], a[0] ^ b[1], a[1] ^ b[1]};
#pragma unroll
  for (int k = 0; k < 8; k++) idx[k] = ab[k & 3] ^ c[k >> 2];
}

// Dense levels have res1^3 <= the level size < 2^32, so res1, res1^2 and the
// cell coordinates fit 24 bits: two v_mad_u32_u24 instead of v_mul_lo_u32.
__device__ __forceinline__ void dense_corners(const uint32_t g[3], uint32_t res1, uint32_t r2, uint32_t idx[8]) {
  const uint32_t base = g[0] + __umul24(g[1], res1) + __umul24(g[2], r2);
#pragma unroll
  for (int k = 0; k < 8; k++) idx[k] = base + ((k & 1) ? 1u : 0u) + ((k & 2) ? res1 : 0u) + ((k & 4) ? r2 : 0u);
}

// Any level layout: the level's flags pick hashed or dense indexing and the
// modulo (none, power-of-two mask, or %).
template <int F, bool kHalf>
__device__ __forceinline__ void level_corners(const LevelTable& lv, int l, float pos_offset, uint32_t interp,
                                              const float u[3], LevelCorners& cn) {
  const uint32_t res1 = lv.res1[l];
  const uint32_t hsize = lv.hsize[l];
  const uint32_t flags = lv.flags[l];
  cn.soff = lv.base[l] * (uint32_t)(F * (kHalf ? 2 : 4));
  cn.dense = 0u;
  uint32_t g[3];
  cell_weights(lv.scale[l], pos_offset, interp == 1, u, g, cn);
  uint32_t* idx = cn.idx;
  if (flags & kLvHashed)
    hashed_corners(g, idx);
  else
    dense_corners(g, res1, res1 * res1, idx);
  if (!(flags & kLvNoMod)) {
    if (flags & kLvPow2) {
#pragma unroll
      for (int k = 0; k < 8; k++) idx[k] &= hsize - 1u;
    } else {
#pragma unroll
      for (int k = 0; k < 8; k++) idx[k] %= hsize;
    }
  }
}

// cell_weights for a looked-up render hit: its grid coordinate u is in
// [0, 1] (the contraction maps into [0, 1], and out-of-range hits of the
// affine normalisation look nothing up), and the caller's pos_offset is 0.5
// (the host sends align_corners grids to the general path), so
// x = u * scale + 0.5 is positive even if the contraction's rounding left u a
// few ulp below 0, and x - (float)f2u_sat(x) is exactly fract(x): one
// v_fract_f32 instead of a conversion back and a subtraction (NaN stays NaN).
__device__ __forceinline__ void cell_weights_unit(float scale, float pos_offset, const float u[3], uint32_t g[3],
                                                  LevelCorners& cn) {
  float pos[3];
#pragma unroll
  for (int d = 0; d < 3; d++) {
    const float x = u[d] * scale + pos_offset;
    g[d] = f2u_sat(x);
    pos[d] = __builtin_amdgcn_fractf(x);
  }
  cn.wx[0] = 1 - pos[0]; cn.wx[1] = pos[0];
  cn.wy[0] = 1 - pos[1]; cn.wy[1] = pos[1];
  cn.wz[0] = 1 - pos[2]; cn.wz[1] = pos[2];
}

// The common grid (levels [0, n_dense) dense with no modulo, the rest hashed
// into power-of-two sizes, trilinear weights) from the level's 16-byte
// record: one uniform test of q.b picks the index path.
__device__ __forceinline__ void quad_corners(const LevelQuad& q, float pos_offset, const float u[3], LevelCorners& cn) {
  cn.soff = q.soff;
  cn.dense = q.b;
  uint32_t g[3];
  cell_weights_unit(q.scale, pos_offset, u, g, cn);
  if (q.b != 0) {
    dense_corners(g, q.a, q.b, cn.idx);
  } else {
    hashed_corners(g, cn.idx);
#pragma unroll
    for (int k = 0; k < 8; k++) cn.idx[k] &= q.a;
  }
}

// Loads the eight corner entries of cn.
template <int F, bool kHalf>
__device__ __forceinline__ void corners_load(nest_i32x4 rsrc, const LevelCorners& cn, float vals[8][F]) {
#pragma unroll
  for (int k = 0; k < 8; k++) struct_entry<F, kHalf>(rsrc, cn.idx[k], cn.soff, vals[k]);
}

// quad_corners followed by corners_load_r in one uniform branch, for the
// common grid with 8-byte entries: a dense level computes only the four
// x-pair bases and issues four 16-byte loads; a hashed level issues eight
// 8-byte loads.  Either way the pair of corners 2m, 2m + 1 lands in one
// 4-dword tuple.
template <int F, bool kHalf>
__device__ __forceinline__ void quad_fetch_pairs(const LevelQuad& q, float pos_offset, const float u[3],
                                                 nest_i32x4 rsrc, LevelCorners& cn, float vals[8][F]) {
  static_assert((kHalf && F == 4) || (!kHalf && F == 2), "8-byte entries");
  cn.soff = q.soff;
  cn.dense = q.b;
  uint32_t g[3];
  cell_weights_unit(q.scale, pos_offset, u, g, cn);
  nest_i32x4 pr[4];
  if (q.b != 0) {
    const nest_i32x4 raw = table_rsrc_raw<F, kHalf>(rsrc);
    const uint32_t base = g[0] + __umul24(g[1], q.a) + __umul24(g[2], q.b);
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const uint32_t e = base + ((m & 1) ? q.a : 0u) + ((m & 2) ? q.b : 0u);
      pr[m] = nest_raw_load_v4i32(raw, (int)(e * 8u), (int)q.soff, 0);
    }
  } else {
    hashed_corners(g, cn.idx);
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const nest_i32x2 a = nest_struct_load_v2i32(rsrc, (int)(cn.idx[2 * m] & q.a), 0, (int)q.soff, 0);
      const nest_i32x2 b = nest_struct_load_v2i32(rsrc, (int)(cn.idx[2 * m + 1] & q.a), 0, (int)q.soff, 0);
      pr[m] = nest_i32x4{a.x, a.y, b.x, b.y};
    }
  }
#pragma unroll
  for (int m = 0; m < 4; m++) {
    vals[2 * m][0] = __int_as_float(pr[m].x);
    vals[2 * m][1] = __int_as_float(pr[m].y);
    vals[2 * m + 1][0] = __int_as_float(pr[m].z);
    vals[2 * m + 1][1] = __int_as_float(pr[m].w);
  }
}

// Interpolated value: out = fmaf(w_k, entry_k, out) over corners 0..7 in
// order, out starting at 0.
template <int F>
__device__ __forceinline__ void corners_sum(const LevelCorners& cn, const float vals[8][F], float out[F]) {
#pragma unroll
  for (int f = 0; f < F; f++) out[f] = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float w = (1.0f * cn.wx[k & 1]) * cn.wy[(k >> 1) & 1] * cn.wz[k >> 2];
#pragma unroll
    for (int f = 0; f < F; f++) out[f] = fmaf(w, vals[k][f], out[f]);
  }
}

// Render path of binary16 tables (F = 2 or 4): the corner entries stay
// packed (two halves per 32-bit word, bit patterns kept in the float array)
// and each interpolation step widens its half inside the FMA with
// v_fma_mix_f32, instead of one v_cvt_f32_f16 per value before it.  The
// widening is exact and the FMA rounds once, so the result is fmaf(w, h, out)
// bit for bit; the mix instruction's float32-denormal flush cannot apply,
// since a product of the cell weights (0, or at least ~1e-21) and a binary16
// value (0, or at least ~6e-8) is never a float32 denormal.
//
// Tables of 8-byte entries (binary16 F = 4, binary32 F = 2): on a dense
// level corners 2m and 2m + 1 (x and x + 1) are neighbouring entries, so one
// 16-byte load from the byte view fetches both, four loads per level instead
// of eight; the values and their order are the same.
template <int F, bool kHalf>
__device__ __forceinline__ void corners_load_r(nest_i32x4 rsrc, const LevelCorners& cn, float vals[8][F]) {
  constexpr bool kPair = (kHalf && F == 4) || (!kHalf && F == 2);
  if constexpr (kPair) {
    // Both branches leave an x-pair in one 4-dword tuple, so the registers
    // the loads land in are the same on either side of the uniform branch.
    nest_i32x4 pr[4];
    if (cn.dense != 0u) {
      const nest_i32x4 raw = table_rsrc_raw<F, kHalf>(rsrc);
#pragma unroll
      for (int m = 0; m < 4; m++) pr[m] = nest_raw_load_v4i32(raw, (int)(cn.idx[2 * m] * 8u), (int)cn.soff, 0);
    } else {
#pragma unroll
      for (int m = 0; m < 4; m++) {
        const nest_i32x2 a = nest_struct_load_v2i32(rsrc, (int)cn.idx[2 * m], 0, (int)cn.soff, 0);
        const nest_i32x2 b = nest_struct_load_v2i32(rsrc, (int)cn.idx[2 * m + 1], 0, (int)cn.soff, 0);
        pr[m] = nest_i32x4{a.x, a.y, b.x, b.y};
      }
    }
#pragma unroll
    for (int m = 0; m < 4; m++) {
      vals[2 * m][0] = __int_as_float(pr[m].x);
      vals[2 * m][1] = __int_as_float(pr[m].y);
      vals[2 * m + 1][0] = __int_as_float(pr[m].z);
      vals[2 * m + 1][1] = __int_as_float(pr[m].w);
    }
    return;
  }
  if constexpr (kHalf && (F == 4 || F == 2)) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      if constexpr (F == 4) {
        const nest_i32x2 a = nest_struct_load_v2i32(rsrc, (int)cn.idx[k], 0, (int)cn.soff, 0);
        vals[k][0] = __int_as_float(a.x);  // channels 0-1; [2], [3] stay unused
        vals[k][1] = __int_as_float(a.y);  // channels 2-3
      } else {
        vals[k][0] = __int_as_float(nest_struct_load_i32(rsrc, (int)cn.idx[k], 0, (int)cn.soff, 0));
      }
    }
  } else {
    corners_load<F, kHalf>(rsrc, cn, vals);
  }
}

__device__ __forceinline__ float fma_mix_lo(float w, float packed, float acc) {
  asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(w), "v"(packed));
  return acc;
}

__device__ __forceinline__ float fma_mix_hi(float w, float packed, float acc) {
  asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(w), "v"(packed));
  return acc;
}

template <int F, bool kHalf>
__device__ __forceinline__ void corners_sum_r(const LevelCorners& cn, const float vals[8][F], float out[F]) {
  if constexpr (kHalf && (F == 4 || F == 2)) {
#pragma unroll
    for (int f = 0; f < F; f++) out[f] = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float w = (1.0f * cn.wx[k & 1]) * cn.wy[(k >> 1) & 1] * cn.wz[k >> 2];
#pragma unroll
      for (int f = 0; f < F; f++)
        out[f] = (f & 1) ? fma_mix_hi(w, vals[k][f >> 1], out[f]) : fma_mix_lo(w, vals[k][f >> 1], out[f]);
    }
  } else {
    corners_sum<F>(cn, vals, out);
  }
}

}  // namespace nest
