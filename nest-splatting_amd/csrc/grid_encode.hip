// Standalone multi-level hash encoding (GridEncoder.forward).
//
// Semantics: kernel_grid / get_grid_index / fast_hash of
// gridencoder/src/gridencoder.cu:50-242 for D in 2..5, gridtype hash (0) or
// tiled (1), float32 or float16 embeddings (float16 accumulates in float16 as
// the reference's scalar_t accumulator does).  The reference writes [L, B, C]
// and permutes to [B, L*C] in Python (gridencoder/grid.py:47, :59); this
// kernel writes [B, L*C] directly.
//
// Lane mapping: consecutive lanes take consecutive levels of the same point,
// so the 4*L..16*L output bytes of a point are one contiguous store run.
#include <hip/hip_fp16.h>

#include "hashgrid.h"
#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }
__device__ __forceinline__ float round_half(float x) { return __half2float(__float2half_rn(x)); }

template <int D, int C, bool kHalf>
__global__ void __launch_bounds__(256) grid_encode_kernel(const GridEncodeParams p) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = t / p.L;
  const int l = (int)(t - b * p.L);
  if (b >= p.B) return;
  const float* in = p.inputs + b * D;
  float u[D];
  bool oob = false;
#pragma unroll
  for (int d = 0; d < D; d++) {
    u[d] = in[d];
    if (u[d] < 0 || u[d] > 1) oob = true;
  }
  float acc[C];
#pragma unroll
  for (int c = 0; c < C; c++) acc[c] = 0.0f;
  if (!oob) {
    const float scale = p.lv.scale[l];
    const uint32_t res1 = p.lv.res1[l];
    const uint32_t hsize = p.lv.hsize[l];
    const uint32_t flags = p.lv.flags[l];
    const uint32_t ndims = (flags >> 8) & 0xffu;
    const size_t base = p.lv.base[l];
    const float off = p.align_corners ? 0.0f : 0.5f;
    float pos[D];
    uint32_t g[D];
#pragma unroll
    for (int d = 0; d < D; d++) {
      pos[d] = u[d] * scale + off;
      g[d] = f2u_sat(pos[d]);  // == f2u_sat(floorf(pos[d]))
      pos[d] = pos[d] - (float)g[d];
      if (p.interp == 1) pos[d] = pos[d] * pos[d] * (3.0f - 2.0f * pos[d]);
    }
    constexpr uint32_t primes[7] = {1u, 2654435761u, 805459861u, 3674653429u, 2097192037u, 1434869437u, 2165219737u};
#pragma unroll
    for (int c = 0; c < (1 << D); c++) {
      float w = 1.0f;
      uint32_t q[D];
#pragma unroll
      for (int d = 0; d < D; d++) {
        if ((c & (1 << d)) == 0) {
          w *= 1 - pos[d];
          q[d] = g[d];
        } else {
          w *= pos[d];
          q[d] = g[d] + 1u;
        }
      }
      uint32_t idx = 0;
      if (flags & kLvHashed) {
#pragma unroll
        for (int d = 0; d < D; d++) idx ^= q[d] * primes[d];
      } else {
        uint32_t stride = 1;
#pragma unroll
        for (int d = 0; d < D; d++) {
          if ((uint32_t)d < ndims) {
            idx += q[d] * stride;
            stride *= res1;
          }
        }
      }
      if (!(flags & kLvNoMod)) idx = (flags & kLvPow2) ? (idx & (hsize - 1u)) : (idx % hsize);
      float v[C];
      load_entry<C, kHalf>(p.table, base + idx, v);
#pragma unroll
      for (int ch = 0; ch < C; ch++) {
        if constexpr (kHalf) {
          // at::Half += float: the float32 product is rounded to float32 and
          // then to float16.  The empty asm keeps the product a float32
          // value; without it the backend folds multiply and conversion into
          // one v_fma_mixlo_f16 with a single rounding.
          float prod = w * v[ch];
          asm volatile("" : "+v"(prod));
          acc[ch] = round_half(acc[ch] + round_half(prod));
        } else {
          acc[ch] = fmaf(w, v[ch], acc[ch]);
        }
      }
    }
  }
  const int64_t o = (b * p.L + l) * C;
  if constexpr (kHalf) {
    __half* out = static_cast<__half*>(p.outputs) + o;
#pragma unroll
    for (int ch = 0; ch < C; ch++) out[ch] = __float2half_rn(acc[ch]);
  } else {
    float* out = static_cast<float*>(p.outputs) + o;
#pragma unroll
    for (int ch = 0; ch < C; ch++) out[ch] = acc[ch];
  }
}

template <int D, bool kHalf>
static hipError_t ge_launch_c(const GridEncodeParams& p, hipStream_t s) {
  const int64_t n = p.B * p.L;
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (p.C) {
    case 1: hipLaunchKernelGGL((grid_encode_kernel<D, 1, kHalf>), grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL((grid_encode_kernel<D, 2, kHalf>), grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL((grid_encode_kernel<D, 4, kHalf>), grid, dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL((grid_encode_kernel<D, 8, kHalf>), grid, dim3(256), 0, s, p); break;
    case 16: hipLaunchKernelGGL((grid_encode_kernel<D, 16, kHalf>), grid, dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <bool kHalf>
static hipError_t ge_launch_d(const GridEncodeParams& p, hipStream_t s) {
  switch (p.D) {
    case 2: return ge_launch_c<2, kHalf>(p, s);
    case 3: return ge_launch_c<3, kHalf>(p, s);
    case 4: return ge_launch_c<4, kHalf>(p, s);
    case 5: return ge_launch_c<5, kHalf>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// Common level layout (D = 3, binary32, trilinear; see GridEncodeQuadParams).
// A workgroup encodes 64 points per iteration: lane = point, and wave w
// takes levels w, w + 4, ..., so each level's record is one scalar load and
// its dense-or-hashed branch is uniform.  A level is quad_corners (or, for
// 8-byte entries, quad_fetch_pairs) and corners_sum, the render's lookup,
// whose float order is kernel_grid's: w = ((1 * w_x) * w_y) * w_z and
// out = fmaf(w, v, out) over corners 0..7 from +0 (inputs are in [0, 1] past
// the range test, so fract(x) is x - floor(x)).  The 64 points' outputs are
// staged in LDS (rows padded by 4 floats against bank conflicts) and written
// as one contiguous run.
constexpr int kGeqThreads = 256;
constexpr int kGeqPoints = 64;

template <int F>
__global__ void __launch_bounds__(kGeqThreads) grid_encode_quad_kernel(const GridEncodeQuadParams p) {
  extern __shared__ float geq_rows[];  // [64][L * F + 4]
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int LF = p.L * F;
  const int ld = LF + 4;
  const nest_i32x4 rsrc = table_rsrc_rows<F, false>(p.table, p.table_rows);
  const int64_t nblk = (p.B + kGeqPoints - 1) / kGeqPoints;
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int64_t b = blk * kGeqPoints + lane;
    float u[3] = {0.0f, 0.0f, 0.0f};
    bool skip = b >= p.B;
    if (!skip) {
      const float* in = p.inputs + 3 * b;
#pragma unroll
      for (int d = 0; d < 3; d++) {
        u[d] = in[d];
        if (u[d] < 0 || u[d] > 1) skip = true;  // outside the grid: every level is zero
      }
    }
    float* row = geq_rows + lane * ld;
    for (int l = wid; l < p.L; l += kGeqThreads / 64) {
      const LevelQuad q = p.lq[l];
      float v[F];
#pragma unroll
      for (int f = 0; f < F; f++) v[f] = 0.0f;
      if (!skip) {
        LevelCorners cn;
        float vals[8][F];
        if constexpr (F == 2) {
          quad_fetch_pairs<2, false>(q, p.pos_offset, u, rsrc, cn, vals);
        } else {
          quad_corners(q, p.pos_offset, u, cn);
          corners_load<F, false>(rsrc, cn, vals);
        }
        corners_sum<F>(cn, vals, v);
      }
#pragma unroll
      for (int f = 0; f < F; f++) row[l * F + f] = v[f];
    }
    __syncthreads();
    const int64_t n0 = blk * kGeqPoints;
    const int pts = (int)(p.B - n0 < kGeqPoints ? p.B - n0 : kGeqPoints);
    float* out = p.outputs + n0 * LF;
    const int total = pts * LF;
    if ((LF & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
      for (int i = 4 * (int)threadIdx.x; i < total; i += 4 * kGeqThreads) {
        const int pt = i / LF, c = i - pt * LF;
        const float* r = geq_rows + pt * ld + c;
        *reinterpret_cast<float4*>(out + i) = make_float4(r[0], r[1], r[2], r[3]);
      }
    } else {
      for (int i = threadIdx.x; i < total; i += kGeqThreads) {
        const int pt = i / LF;
        out[i] = geq_rows[pt * ld + (i - pt * LF)];
      }
    }
    __syncthreads();
  }
}

hipError_t launch_grid_encode_quad(const GridEncodeQuadParams& p, hipStream_t s) {
  if (p.B <= 0) return hipSuccess;
  const int64_t nblk = (p.B + kGeqPoints - 1) / kGeqPoints;
  const unsigned blocks = (unsigned)(nblk < 4096 ? nblk : 4096);
  const size_t lds = sizeof(float) * (size_t)kGeqPoints * (size_t)(p.L * p.F + 4);
  switch (p.F) {
    case 1: hipLaunchKernelGGL(grid_encode_quad_kernel<1>, dim3(blocks), dim3(kGeqThreads), lds, s, p); break;
    case 2: hipLaunchKernelGGL(grid_encode_quad_kernel<2>, dim3(blocks), dim3(kGeqThreads), lds, s, p); break;
    case 4: hipLaunchKernelGGL(grid_encode_quad_kernel<4>, dim3(blocks), dim3(kGeqThreads), lds, s, p); break;
    case 8: hipLaunchKernelGGL(grid_encode_quad_kernel<8>, dim3(blocks), dim3(kGeqThreads), lds, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_grid_encode(const GridEncodeParams& p, hipStream_t s) {
  if (p.B <= 0) return hipSuccess;
  return p.half ? ge_launch_d<true>(p, s) : ge_launch_d<false>(p, s);
}

}  // namespace nest
