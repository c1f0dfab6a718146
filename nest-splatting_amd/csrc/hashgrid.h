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

__device__ __forceinline__ uint32_t level_index(uint32_t flags, uint32_t res1, uint32_t hsize, uint32_t q0, uint32_t q1,
                                                uint32_t q2) {
  uint32_t idx;
  if (flags & kLvHashed) {
    idx = (q0 * 1u) ^ (q1 * 2654435761u) ^ (q2 * 805459861u);
  } else {
    idx = q0;
    idx += q1 * res1;
    idx += q2 * (res1 * res1);
  }
  if (flags & kLvNoMod) return idx;
  if (flags & kLvPow2) return idx & (hsize - 1u);
  return idx % hsize;
}

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

// Trilinear (interp 0) or smoothstep (interp 1) interpolation of level l at
// u in [0,1]^3.  out[f] = sum over corners 0..7 of w_corner * table, summed
// in corner order from +0, as the reference's results[] accumulator.
template <int F, bool kHalf>
__device__ __forceinline__ void level_interp(const LevelTable& lv, int l, const void* table, float pos_offset,
                                             uint32_t interp, const float u[3], float out[F]) {
  const float scale = lv.scale[l];
  const uint32_t res1 = lv.res1[l];
  const uint32_t hsize = lv.hsize[l];
  const uint32_t flags = lv.flags[l];
  const size_t base = lv.base[l];
  float pos[3];
  uint32_t g[3];
#pragma unroll
  for (int d = 0; d < 3; d++) {
    pos[d] = u[d] * scale + pos_offset;
    g[d] = f2u_sat(floorf(pos[d]));
    pos[d] = pos[d] - (float)g[d];
    if (interp == 1) pos[d] = pos[d] * pos[d] * (3.0f - 2.0f * pos[d]);
  }
#pragma unroll
  for (int f = 0; f < F; f++) out[f] = 0.0f;
  // issue all eight gathers before consuming them
  uint32_t idx[8];
  float wts[8];
#pragma unroll
  for (int c = 0; c < 8; c++) {
    float w = 1.0f;
    w *= (c & 1) ? pos[0] : 1 - pos[0];
    w *= (c & 2) ? pos[1] : 1 - pos[1];
    w *= (c & 4) ? pos[2] : 1 - pos[2];
    wts[c] = w;
    idx[c] = level_index(flags, res1, hsize, g[0] + ((c & 1) ? 1u : 0u), g[1] + ((c & 2) ? 1u : 0u),
                         g[2] + ((c & 4) ? 1u : 0u));
  }
  float vals[8][F];
#pragma unroll
  for (int c = 0; c < 8; c++) load_entry<F, kHalf>(table, base + idx[c], vals[c]);
#pragma unroll
  for (int c = 0; c < 8; c++) {
#pragma unroll
    for (int f = 0; f < F; f++) out[f] += wts[c] * vals[c][f];
  }
}

}  // namespace nest
