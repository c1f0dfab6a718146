// Device math shared by the gfx950 kernels of the forward render.
//
// Every kernel of this library is compiled with -ffp-contract=off, so each
// a*b+c below is a rounded multiply followed by a rounded add, evaluated in the
// order the reference writes it (submodules/diff-surfel-rasterization/
// cuda_rasterizer/forward.cu and hashgrid.h).  Division and sqrtf are the
// correctly rounded HIP defaults.  The exponential is nest_expf(), not the
// device library's, so that the hit/miss decisions of the alpha test
// (alpha >= 1/255, T*(1-alpha) >= 1e-4) are reproducible bit for bit on any
// IEEE-754 host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nest {

// exp(x) in binary32: Cody-Waite reduction x = k ln2 + r with a 9-bit head of
// ln2 (exact k*head for |k| < 2^15), degree-5 minimax polynomial on
// |r| <= ln2/2 (Moshier, Methods and Programs for Mathematical Functions,
// 1989), scaling by 2^k through the exponent field.  x < -87 returns 0,
// x > 88 returns +inf, NaN propagates.
__device__ __forceinline__ float expf_ref(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return __int_as_float(0x7f800000);
  const float t = x * 1.44269504088896341f;
  const float fk = floorf(t + 0.5f);
  float r = x - fk * 0.693359375f;
  r = r - fk * -2.12194440e-4f;
  const float z = r * r;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  const float y = p * z + r + 1.0f;
  const int k = (int)fk;
  return y * __int_as_float((k + 127) << 23);
}

// log(x) in binary32 (Moshier, Methods and Programs for Mathematical
// Functions, 1989): x = m 2^e with m in [sqrt(1/2), sqrt(2)), f = m - 1,
// log(1 + f) = f - f^2/2 + f^3 P(f) with a degree-8 minimax P, plus e ln2 in
// a 9-bit head and a tail.  0 gives -inf, negatives NaN, +inf and NaN
// themselves; subnormals are scaled by 2^23 first.
__device__ __forceinline__ float logf_ref(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? __int_as_float(0xff800000) : __int_as_float(0x7fc00000);
  if (x == __int_as_float(0x7f800000)) return x;
  uint32_t u = __float_as_uint(x);
  int e = 0;
  if (u < 0x00800000u) {
    u = __float_as_uint(x * 8388608.0f);
    e = -23;
  }
  e += (int)((u >> 23) & 0xffu) - 126;
  float m = __uint_as_float((u & 0x007fffffu) | 0x3f000000u);  // [0.5, 1)
  if (m < 0.707106781186547524f) {
    e -= 1;
    m = m + m - 1.0f;
  } else {
    m = m - 1.0f;
  }
  const float z = m * m;
  float y = 7.0376836292e-2f;
  y = y * m + -1.1514610310e-1f;
  y = y * m + 1.1676998740e-1f;
  y = y * m + -1.2420140846e-1f;
  y = y * m + 1.4249322787e-1f;
  y = y * m + -1.6668057665e-1f;
  y = y * m + 2.0000714765e-1f;
  y = y * m + -2.4999993993e-1f;
  y = y * m + 3.3333331174e-1f;
  y = y * m * z;
  const float fe = (float)e;
  y = y + -2.12194440e-4f * fe;
  y = y + -0.5f * z;
  float r = m + y;
  r = r + 0.693359375f * fe;
  return r;
}

// x^y for x >= 0 as expf_ref(y * logf_ref(x)); y == 0 gives 1 (0^0 and
// NaN^0 included), 0^y 0 for y > 0 and +inf for y < 0.  Not correctly
// rounded: the relative error grows with |y log x| (about 5e-6 at 88).
__device__ __forceinline__ float powf_ref(float x, float y) {
  if (y == 0.0f) return 1.0f;
  return expf_ref(y * logf_ref(x));
}

// float -> int with the operand clamped to +-2^30 first (NaN -> -2^30 through
// fmaxf), so the conversion never leaves the representable range.
__device__ __forceinline__ int f2i_sat(float x) {
  x = fmaxf(x, -1073741824.0f);
  x = fminf(x, 1073741824.0f);
  return (int)x;
}

// float -> uint32 truncation; negatives and NaN give 0, 2^32 and above give
// 0xFFFFFFFF.  v_cvt_u32_f32 clamps exactly so (a C cast of an out-of-range
// value is undefined, and the guarded C form compiles to branches).  Since
// truncation equals floor for x >= 0 and both sides give 0 below,
// f2u_sat(x) == f2u_sat(floorf(x)) for every x.
__device__ __forceinline__ uint32_t f2u_sat(float x) {
  uint32_t r;
  asm("v_cvt_u32_f32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

__device__ __forceinline__ uint32_t clamp_tile(int v, uint32_t g) {
  return v < 0 ? 0u : ((uint32_t)v < g ? (uint32_t)v : g);
}

// getRect (cuda_rasterizer/auxiliary.h:72-82) for 16x16 tiles.  The upper
// bound "p + r + BLOCK - 1" associates as ((p + r) + 16) - 1 in float.
__device__ __forceinline__ void tile_rect(float px, float py, int r, uint32_t gx, uint32_t gy,
                                          uint32_t& x0, uint32_t& y0, uint32_t& x1, uint32_t& y1) {
  const float fr = (float)r;
  x0 = clamp_tile(f2i_sat((px - fr) / 16.0f), gx);
  y0 = clamp_tile(f2i_sat((py - fr) / 16.0f), gy);
  x1 = clamp_tile(f2i_sat((px + fr + 16.0f - 1.0f) / 16.0f), gx);
  y1 = clamp_tile(f2i_sat((py + fr + 16.0f - 1.0f) / 16.0f), gy);
}

}  // namespace nest
