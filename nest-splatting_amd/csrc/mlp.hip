// View-direction MLP decode of the composited feature map.
//
// Semantics: INGP.get_color / rgb_decode (hash_encoder/modules.py:587-602):
// x = [feature (C), SH16((d+1)/2)] -> ReLU(W1 x) -> ReLU(W2 .) -> W3 . (no
// biases, HE:560-572) -> sigmoid -> first 3 outputs, then the mask and
// background of gaussian_renderer/__init__.py:1013-1021.  View directions are
// cam2rays (utils/point_utils.py:31-46) normalised, evaluated per pixel from a
// 3x3 matrix so no ray buffer is read.  The SH basis is the degree-3 real SH
// (16 terms) of the SphericalHarmonics encoding (HE:551-558), evaluated on
// 2u-1 of the encoder input u = (d+1)/2.
//
// MFMA formulation (f16 / bf16, fp32 accumulate), one 64-lane wave per 16
// pixels: every layer computes Y^T = W X^T with v_mfma_f32_16x16x16, A = the
// weights (LDS, padded rows), B = the activations.  The accumulator layout of
// 16x16x16 (lane l holds rows 4*(l/16)..+3 of column l%16) is exactly the B
// operand layout of the next layer's K-chunk, so hidden activations never
// leave registers: ReLU, round to 16 bits, feed.
#include <hip/hip_fp16.h>

#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// Round to nearest even: one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint16_t to_bf16_rne(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ uint16_t to_f16_rne(float f) { return __half_as_ushort(__float2half_rn(f)); }

template <bool kBF16>
__device__ __forceinline__ uint16_t to16(float f) {
  if constexpr (kBF16) return to_bf16_rne(f);
  else return to_f16_rne(f);
}

template <bool kBF16>
__device__ __forceinline__ f32x4 mfma16(uint2 a, uint2 b, f32x4 c) {
  if constexpr (kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ uint2 pack4(uint16_t a, uint16_t b, uint16_t c, uint16_t d) {
  return make_uint2((uint32_t)a | ((uint32_t)b << 16), (uint32_t)c | ((uint32_t)d << 16));
}

__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) { return (uint32_t)a | ((uint32_t)b << 16); }

typedef __bf16 nest_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 nest_f16x2 __attribute__((ext_vector_type(2)));
typedef float nest_f32x2v __attribute__((ext_vector_type(2)));
typedef short nest_i16x2 __attribute__((ext_vector_type(2)));

// Two floats as a packed pair (a in the low half), rounded to nearest even:
// one v_cvt_pk_bf16_f32 or v_cvt_pk_f16_f32.
template <bool kBF16>
__device__ __forceinline__ uint32_t pack2_16(float a, float b) {
  if constexpr (kBF16) {
    const nest_bf16x2 h = __builtin_convertvector((nest_f32x2v){a, b}, nest_bf16x2);
    return __builtin_bit_cast(uint32_t, h);
  } else {
    const nest_f16x2 h = __builtin_convertvector((nest_f32x2v){a, b}, nest_f16x2);
    return __builtin_bit_cast(uint32_t, h);
  }
}

// max(a, 0), max(b, 0) as a packed 16-bit float pair: rounding first and
// then replacing every half whose sign bit is set (a negative value or -0)
// by +0, a signed 16-bit maximum with 0 on both halves at once, gives the
// same bits for finite inputs (rounding to nearest keeps the sign, and a
// negative value never rounds to +0).
template <bool kBF16>
__device__ __forceinline__ uint32_t relu_pack2(float a, float b) {
  const nest_i16x2 h = __builtin_bit_cast(nest_i16x2, pack2_16<kBF16>(a, b));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(h, (nest_i16x2){0, 0}));
}


// Raw buffer view of the feature map: per-lane byte offset in a VGPR, the
// channel's byte offset in an SGPR, so the 64 loads of a tile need no
// per-channel 64-bit addresses.
typedef int mlp_i32x4 __attribute__((ext_vector_type(4)));
__device__ float mlp_raw_load_f32(mlp_i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.f32");

__device__ __forceinline__ mlp_i32x4 feat_rsrc(const float* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  mlp_i32x4 r;
  r.x = (int)(uint32_t)(a & 0xffffffffu);
  r.y = (int)(uint32_t)((a >> 32) & 0xffffu);  // stride 0: raw addressing
  r.z = (int)0xffffffffu;                      // range in bytes
  r.w = 0x00020000;
  return r;
}

// The C features of pixel nn (channel c at byte c * cs4 + nn * ns4).
template <int C>
__device__ __forceinline__ void load_features(mlp_i32x4 rsrc, uint32_t cs4, uint32_t voff, float f[C]) {
#pragma unroll
  for (int c = 0; c < C; c++) f[c] = mlp_raw_load_f32(rsrc, (int)voff, (int)(cs4 * (uint32_t)c), 0);
}

// Unit view direction of pixel n of a width-w image: cam2rays rows (x, y, 1) @ M,
// normalised (32-bit pixel arithmetic; the image has fewer than 2^31 pixels).
__device__ __forceinline__ void pixel_dir32(const MlpParams& p, uint32_t n, float& dx, float& dy, float& dz) {
  if (p.dirs) {
    dx = p.dirs[3 * (size_t)n + 0];
    dy = p.dirs[3 * (size_t)n + 1];
    dz = p.dirs[3 * (size_t)n + 2];
    return;
  }
  const uint32_t w = (uint32_t)p.img_w;
  const uint32_t yi = n / w;
  const float x = (float)(n - yi * w), y = (float)yi;
  const float* M = p.M;
  const float rx = x * M[0] + y * M[3] + M[6];
  const float ry = x * M[1] + y * M[4] + M[7];
  const float rz = x * M[2] + y * M[5] + M[8];
  // 1 / max(|r|, 1e-12) as one hardware reciprocal square root (~1 ulp)
  const float il = fminf(__builtin_amdgcn_rsqf(rx * rx + ry * ry + rz * rz), 1e12f);
  dx = rx * il;
  dy = ry * il;
  dz = rz * il;
}

// Hidden unit of slot q = 32 kc + 8 grp + i of a K-chunk built from two
// accumulator M-tiles.
__device__ __forceinline__ int hidden_unit(int q) {
  const int kc = q >> 5, r = q & 31, grp = r >> 3, i = r & 7;
  return 32 * kc + (i < 4 ? 4 * grp + i : 16 + 4 * grp + (i - 4));
}


// SH16 of the unit direction d, computed on x = 2u - 1 with u = (d + 1) / 2.
__device__ __forceinline__ void sh16(float dx, float dy, float dz, float o[16]) {
  const float ux = (dx + 1.0f) / 2.0f, uy = (dy + 1.0f) / 2.0f, uz = (dz + 1.0f) / 2.0f;
  const float x = ux * 2.0f - 1.0f, y = uy * 2.0f - 1.0f, z = uz * 2.0f - 1.0f;
  const float xy = x * y, xz = x * z, yz = y * z, x2 = x * x, y2 = y * y, z2 = z * z;
  o[0] = 0.28209479177387814f;
  o[1] = -0.48860251190291987f * y;
  o[2] = 0.48860251190291987f * z;
  o[3] = -0.48860251190291987f * x;
  o[4] = 1.0925484305920792f * xy;
  o[5] = -1.0925484305920792f * yz;
  o[6] = 0.94617469575755997f * z2 - 0.31539156525251999f;
  o[7] = -1.0925484305920792f * xz;
  o[8] = 0.54627421529603959f * x2 - 0.54627421529603959f * y2;
  o[9] = 0.59004358992664352f * y * (-3.0f * x2 + y2);
  o[10] = 2.8906114426405538f * xy * z;
  o[11] = 0.45704579946446572f * y * (1.0f - 5.0f * z2);
  o[12] = 0.3731763325901154f * z * (5.0f * z2 - 3.0f);
  o[13] = 0.45704579946446572f * x * (1.0f - 5.0f * z2);
  o[14] = 1.4453057213202769f * z * (x2 - y2);
  o[15] = 0.59004358992664352f * x * (-x2 + 3.0f * y2);
}

__device__ __forceinline__ void pixel_dir(const MlpParams& p, int64_t n, float& dx, float& dy, float& dz) {
  if (p.dirs) {
    dx = p.dirs[3 * n + 0];
    dy = p.dirs[3 * n + 1];
    dz = p.dirs[3 * n + 2];
    return;
  }
  const float x = (float)(n % p.img_w), y = (float)(n / p.img_w);
  const float* M = p.M;
  const float rx = x * M[0] + y * M[3] + M[6];
  const float ry = x * M[1] + y * M[4] + M[7];
  const float rz = x * M[2] + y * M[5] + M[8];
  // 1 / max(|r|, 1e-12) as one hardware reciprocal square root (~1 ulp)
  const float il = fminf(__builtin_amdgcn_rsqf(rx * rx + ry * ry + rz * rz), 1e12f);
  dx = rx * il;
  dy = ry * il;
  dz = rz * il;
}

// Output sigmoid 1 / (1 + 2^(-x log2 e)) on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32; a few ulp, far inside the decode's 1e-3 tolerance):
// four VALU operations where the exact exp and IEEE division take ~30, and
// the output rows of a tile sit on a quarter of the lanes.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

__device__ __forceinline__ float finish_rgb(const MlpParams& p, int64_t n, float logit, int o) {
  float r = sigmoid_fast(logit);
  if (p.alpha) {
    const float a = p.alpha[n];
    r = a > 0.0f ? r : 0.0f;
    if (p.use_bg) r = r + (1.0f - a) * p.bg[o];
  }
  return r;
}

// finish_rgb with the pixel's alpha already loaded (1 when there is no mask).
__device__ __forceinline__ float finish_rgb_alpha(const MlpParams& p, float a, float logit, int o) {
  float r = sigmoid_fast(logit);
  if (p.alpha) {
    r = a > 0.0f ? r : 0.0f;
    if (p.use_bg) r = r + (1.0f - a) * p.bg[o];
  }
  return r;
}

constexpr int kMlpThreads = 256;

// NT = width / 16.  KC1 = ceil((C + 16) / 16) K-chunks in layer 1.  KF > 0:
// C == 16 KF, the features fill KF whole chunks and the SH terms the last
// one; a lane's 4 KF feature loads of a tile are then issued together (one
// load latency per tile instead of one per chunk), and a lane evaluates only
// the 4 SH terms of its row group.
template <int NT, bool kBF16, int KF>
__global__ void __launch_bounds__(kMlpThreads) __attribute__((amdgpu_waves_per_eu(NT <= 4 ? 3 : 1)))
mlp_mfma_kernel(const MlpParams p) {
  extern __shared__ uint16_t lds[];
  const int C = p.C;
  const int KC1 = (C + 16 + 15) / 16;
  const int ld1 = KC1 * 16 + 4, ld2 = NT * 16 + 4, ld3 = NT * 16 + 4;
  uint16_t* w1 = lds;
  uint16_t* w2 = w1 + NT * 16 * ld1;
  uint16_t* w3 = w2 + NT * 16 * ld2;
  const int Kin = C + 16;
  const uint16_t* g1 = static_cast<const uint16_t*>(p.w1);
  const uint16_t* g2 = static_cast<const uint16_t*>(p.w2);
  const uint16_t* g3 = static_cast<const uint16_t*>(p.w3);
  for (int i = threadIdx.x; i < NT * 16 * ld1; i += kMlpThreads) {
    const int r = i / ld1, k = i % ld1;
    w1[i] = k < Kin ? g1[r * Kin + k] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < NT * 16 * ld2; i += kMlpThreads) {
    const int r = i / ld2, k = i % ld2;
    w2[i] = k < NT * 16 ? g2[r * NT * 16 + k] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < 16 * ld3; i += kMlpThreads) {
    const int r = i / ld3, k = i % ld3;
    w3[i] = (r < 3 && k < NT * 16) ? g3[r * NT * 16 + k] : (uint16_t)0;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t ntile = (p.N + 15) / 16;
  const int64_t wave = (int64_t)blockIdx.x * (kMlpThreads / 64) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (kMlpThreads / 64);

  for (int64_t t = wave; t < ntile; t += nwaves) {
    const int64_t n = t * 16 + col;
    const bool valid = n < p.N;
    const int64_t nn = valid ? n : p.N - 1;

    float xf[KF > 0 ? KF : 1][4];
    if constexpr (KF > 0) {
#pragma unroll
      for (int kc = 0; kc < KF; kc++)
#pragma unroll
        for (int i = 0; i < 4; i++) xf[kc][i] = p.feat[(int64_t)(kc * 16 + grp * 4 + i) * p.feat_cs + nn * p.feat_ns];
    }
    float dx, dy, dz;
    pixel_dir(p, nn, dx, dy, dz);
    float sh[16];
    float s4[4];  // KF > 0: the SH terms grp * 4 + i of this lane's row group
    if constexpr (KF > 0) {
      // each branch keeps only its own 4 terms of the inlined basis
      switch (grp) {
        case 0: sh16(dx, dy, dz, sh); s4[0] = sh[0]; s4[1] = sh[1]; s4[2] = sh[2]; s4[3] = sh[3]; break;
        case 1: sh16(dx, dy, dz, sh); s4[0] = sh[4]; s4[1] = sh[5]; s4[2] = sh[6]; s4[3] = sh[7]; break;
        case 2: sh16(dx, dy, dz, sh); s4[0] = sh[8]; s4[1] = sh[9]; s4[2] = sh[10]; s4[3] = sh[11]; break;
        default: sh16(dx, dy, dz, sh); s4[0] = sh[12]; s4[1] = sh[13]; s4[2] = sh[14]; s4[3] = sh[15]; break;
      }
    } else {
      sh16(dx, dy, dz, sh);
    }

    f32x4 acc1[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) acc1[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (KF > 0) {
#pragma unroll
      for (int kc = 0; kc <= KF; kc++) {
        float xv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = kc < KF ? xf[kc < KF ? kc : 0][i] : s4[i];
        const uint2 b = make_uint2(pack2_16<kBF16>(xv[0], xv[1]), pack2_16<kBF16>(xv[2], xv[3]));
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
          const uint2 a = *reinterpret_cast<const uint2*>(w1 + (nt * 16 + col) * ld1 + kc * 16 + grp * 4);
          acc1[nt] = mfma16<kBF16>(a, b, acc1[nt]);
        }
      }
    }
    for (int kc = 0; KF == 0 && kc < KC1; kc++) {
      float xv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int k = kc * 16 + grp * 4 + i;
        if (k < C) {
          xv[i] = p.feat[(int64_t)k * p.feat_cs + nn * p.feat_ns];
        } else {
          const int s = k - C;
          float v = 0.0f;
#pragma unroll
          for (int q = 0; q < 16; q++) v = (s == q) ? sh[q] : v;
          xv[i] = v;
        }
      }
      const uint2 b = make_uint2(pack2_16<kBF16>(xv[0], xv[1]), pack2_16<kBF16>(xv[2], xv[3]));
#pragma unroll
      for (int nt = 0; nt < NT; nt++) {
        const uint2 a = *reinterpret_cast<const uint2*>(w1 + (nt * 16 + col) * ld1 + kc * 16 + grp * 4);
        acc1[nt] = mfma16<kBF16>(a, b, acc1[nt]);
      }
    }
    uint2 h1[NT];
#pragma unroll
    for (int i = 0; i < NT; i++)
      h1[i] = make_uint2(relu_pack2<kBF16>(acc1[i][0], acc1[i][1]), relu_pack2<kBF16>(acc1[i][2], acc1[i][3]));
    f32x4 acc2[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) acc2[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < NT; kc++) {
#pragma unroll
      for (int nt = 0; nt < NT; nt++) {
        const uint2 a = *reinterpret_cast<const uint2*>(w2 + (nt * 16 + col) * ld2 + kc * 16 + grp * 4);
        acc2[nt] = mfma16<kBF16>(a, h1[kc], acc2[nt]);
      }
    }
    f32x4 acc3 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < NT; kc++) {
      const uint2 h2 = make_uint2(relu_pack2<kBF16>(acc2[kc][0], acc2[kc][1]), relu_pack2<kBF16>(acc2[kc][2], acc2[kc][3]));
      const uint2 a = *reinterpret_cast<const uint2*>(w3 + col * ld3 + kc * 16 + grp * 4);
      acc3 = mfma16<kBF16>(a, h2, acc3);
    }
    if (grp == 0 && valid) {
#pragma unroll
      for (int o = 0; o < 3; o++) p.out[o * p.out_os + n * p.out_ns] = finish_rgb(p, n, acc3[o], o);
    }
  }
}

// gfx950 formulation with v_mfma_f32_16x16x32 (bf16 / f16): one wave per 64
// pixels per iteration, for feature maps of 16, 32 or 64 channels and width
// 32 or 64.
//  - Loads: lane = pixel, so every feature load is 64 consecutive pixels of
//    one channel (256 contiguous bytes); the lane rounds its pixel's features
//    and SH terms to 16 bits into a per-wave LDS row [64 px][K1 + 8], K1 =
//    C + 16 rounded up to 32 (zero tail).
//  - Layer 1: B operands are 16-byte LDS reads of that row (pixel col of
//    N-tile j, channels 32 kc + 8 grp .. + 7), A operands the same slice of W1
//    in LDS; A and B put channel 32 kc + 8 grp + i in the same (lane group,
//    element) slot, so the product sums over the chunk's channels.
//  - Layers 2 and 3: the 16x16 accumulator of M-tile mt holds hidden units
//    16 mt + 4 grp + i (i < 4) in lane group grp; K-chunk kc of the next layer
//    takes M-tiles 2 kc and 2 kc + 1, so its slot (grp, i) holds unit
//    32 kc + 4 grp + i (i < 4) or 32 kc + 16 + 4 grp + i - 4 (i >= 4).  The
//    weights are stored in LDS with their columns in that order, so hidden
//    activations stay in registers (ReLU, round to 16 bits, feed).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <bool kBF16>
__device__ __forceinline__ f32x4 mfma32(uint4 a, uint4 b, f32x4 c) {
  if constexpr (kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  }
}


template <bool kBF16>
__device__ __forceinline__ uint4 relu_pack8(f32x4 lo, f32x4 hi) {
  return make_uint4(relu_pack2<kBF16>(lo[0], lo[1]), relu_pack2<kBF16>(lo[2], lo[3]),
                    relu_pack2<kBF16>(hi[0], hi[1]), relu_pack2<kBF16>(hi[2], hi[3]));
}

constexpr int kMlp32Waves = kMlpThreads / 64;

template <int C, int NT>
struct Mlp32Shape {
  static constexpr int K1 = ((C + 16) + 31) / 32 * 32;
  static constexpr int LD1 = K1 + 8;          // halfs per W1 / pixel row (16-byte multiple)
  static constexpr int LD2 = NT * 16 + 8;     // halfs per W2 / W3 row
  static constexpr int W1 = 0;
  static constexpr int W2 = W1 + NT * 16 * LD1;
  static constexpr int W3 = W2 + NT * 16 * LD2;
  static constexpr int X = W3 + 16 * LD2;     // per-wave pixel rows
  static constexpr int TOTAL = X + kMlp32Waves * 64 * LD1;
};

template <int NT, bool kBF16, int C>
__global__ void __launch_bounds__(kMlpThreads) __attribute__((amdgpu_waves_per_eu(2)))
mlp_mfma32_kernel(const MlpParams p) {
  using S = Mlp32Shape<C, NT>;
  constexpr int K1 = S::K1, LD1 = S::LD1, LD2 = S::LD2, W = NT * 16;
  static_assert(NT % 2 == 0, "hidden width must be a multiple of 32");
  extern __shared__ uint16_t lds[];
  uint16_t* w1 = lds + S::W1;
  uint16_t* w2 = lds + S::W2;
  uint16_t* w3 = lds + S::W3;
  const uint16_t* g1 = static_cast<const uint16_t*>(p.w1);
  const uint16_t* g2 = static_cast<const uint16_t*>(p.w2);
  const uint16_t* g3 = static_cast<const uint16_t*>(p.w3);
  constexpr int Kin = C + 16;
  for (int i = threadIdx.x; i < W * LD1; i += kMlpThreads) {
    const int r = i / LD1, k = i % LD1;
    w1[i] = k < Kin ? g1[r * Kin + k] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < W * LD2; i += kMlpThreads) {
    const int r = i / LD2, q = i % LD2;
    w2[i] = q < W ? g2[r * W + hidden_unit(q)] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < 16 * LD2; i += kMlpThreads) {
    const int r = i / LD2, q = i % LD2;
    w3[i] = (r < 3 && q < W) ? g3[r * W + hidden_unit(q)] : (uint16_t)0;
  }
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  uint16_t* xrow = lds + S::X + (threadIdx.x >> 6) * 64 * LD1;  // this wave's 64 pixel rows
  // zero tail of the pixel rows (channels C + 16 .. K1 - 1), written once
  for (int k = Kin; k < K1; k++) xrow[lane * LD1 + k] = 0;
  __syncthreads();

  // pixel indices and byte offsets fit 32 bits (checked by the launcher)
  const uint32_t N = (uint32_t)p.N;
  const uint32_t ntile = (N + 63) / 64;
  const uint32_t wave = blockIdx.x * kMlp32Waves + (threadIdx.x >> 6);
  const uint32_t nwaves = gridDim.x * kMlp32Waves;
  const mlp_i32x4 rsrc = feat_rsrc(p.feat);
  const uint32_t cs4 = (uint32_t)p.feat_cs * 4u, ns4 = (uint32_t)p.feat_ns * 4u;
  // Features and alpha of the tile being processed, loaded during the previous
  // tile (vmcnt counts at most 63 loads in flight, so the next tile's loads
  // are issued only once nothing of this tile is waited for any more).
  float f[C];
  float alpha4[4] = {1.0f, 1.0f, 1.0f, 1.0f};  // lane group 0: its output pixels' alpha
  auto load_tile = [&](uint32_t tt) {
    if (p.alpha && grp == 0) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t nj = tt * 64 + 16 * j + col;
        alpha4[j] = p.alpha[nj < N ? nj : N - 1];
      }
    }
    const uint32_t n0 = tt * 64 + lane;
    load_features<C>(rsrc, cs4, (n0 < N ? n0 : N - 1) * ns4, f);
  };
  if (wave < ntile) load_tile(wave);
  for (uint32_t t = wave; t < ntile; t += nwaves) {
    const uint32_t n = t * 64 + lane;
    const uint32_t nn = n < N ? n : N - 1;
    float dx, dy, dz;
    pixel_dir32(p, nn, dx, dy, dz);
    float sh[16];
    sh16(dx, dy, dz, sh);
    uint4* row4 = reinterpret_cast<uint4*>(xrow + lane * LD1);
#pragma unroll
    for (int q = 0; q < C / 8; q++)
      row4[q] = make_uint4(pack2_16<kBF16>(f[8 * q + 0], f[8 * q + 1]), pack2_16<kBF16>(f[8 * q + 2], f[8 * q + 3]),
                           pack2_16<kBF16>(f[8 * q + 4], f[8 * q + 5]), pack2_16<kBF16>(f[8 * q + 6], f[8 * q + 7]));
#pragma unroll
    for (int q = 0; q < 2; q++)
      row4[C / 8 + q] = make_uint4(pack2_16<kBF16>(sh[8 * q + 0], sh[8 * q + 1]), pack2_16<kBF16>(sh[8 * q + 2], sh[8 * q + 3]),
                                   pack2_16<kBF16>(sh[8 * q + 4], sh[8 * q + 5]), pack2_16<kBF16>(sh[8 * q + 6], sh[8 * q + 7]));
    const float a_out[4] = {alpha4[0], alpha4[1], alpha4[2], alpha4[3]};
    // the next tile's features and alpha are in flight during this tile's contraction
    if (t + nwaves < ntile) load_tile(t + nwaves);
    __builtin_amdgcn_wave_barrier();
    // layer 1: 4 N-tiles of 16 pixels
    f32x4 acc1[NT][4];
#pragma unroll
    for (int mt = 0; mt < NT; mt++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc1[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < K1 / 32; kc++) {
      uint4 b[4];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = *reinterpret_cast<const uint4*>(xrow + (16 * j + col) * LD1 + 32 * kc + 8 * grp);
#pragma unroll
      for (int mt = 0; mt < NT; mt++) {
        const uint4 a = *reinterpret_cast<const uint4*>(w1 + (16 * mt + col) * LD1 + 32 * kc + 8 * grp);
#pragma unroll
        for (int j = 0; j < 4; j++) acc1[mt][j] = mfma32<kBF16>(a, b[j], acc1[mt][j]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the rows are read; the next tile may overwrite them
    // layer 2
    f32x4 acc2[NT][4];
#pragma unroll
    for (int mt = 0; mt < NT; mt++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc2[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < NT / 2; kc++) {
      uint4 b[4];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = relu_pack8<kBF16>(acc1[2 * kc][j], acc1[2 * kc + 1][j]);
#pragma unroll
      for (int mt = 0; mt < NT; mt++) {
        const uint4 a = *reinterpret_cast<const uint4*>(w2 + (16 * mt + col) * LD2 + 32 * kc + 8 * grp);
#pragma unroll
        for (int j = 0; j < 4; j++) acc2[mt][j] = mfma32<kBF16>(a, b[j], acc2[mt][j]);
      }
    }
    // layer 3: rows 0-2 of one M-tile are the RGB logits
    f32x4 acc3[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc3[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < NT / 2; kc++) {
      const uint4 a = *reinterpret_cast<const uint4*>(w3 + col * LD2 + 32 * kc + 8 * grp);
#pragma unroll
      for (int j = 0; j < 4; j++) acc3[j] = mfma32<kBF16>(a, relu_pack8<kBF16>(acc2[2 * kc][j], acc2[2 * kc + 1][j]), acc3[j]);
    }
    if (grp == 0) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t nj = t * 64 + 16 * j + col;
        if (nj < N) {
#pragma unroll
          for (int o = 0; o < 3; o++)
            p.out[o * p.out_os + (int64_t)nj * p.out_ns] = finish_rgb_alpha(p, a_out[j], acc3[j][o], o);
        }
      }
    }
  }
}

// The 16x16x32 kernel addresses pixels and feature bytes with 32 bits.
static bool mlp32_fits(const MlpParams& p, int C) {
  const uint64_t maxoff = ((uint64_t)(C - 1) * (uint64_t)p.feat_cs + (uint64_t)(p.N - 1) * (uint64_t)p.feat_ns) * 4u;
  return p.N < (1ll << 31) - 64 && p.feat_cs >= 0 && p.feat_ns >= 0 && maxoff < 0xffffffffull;
}

// Pixel rows of the block kernel: 16-byte chunk c of row r (a pixel of the
// 256-pixel block) is stored at chunk (c & ~3) | ((c & 3) ^ ((r >> 4) & 3))
// of the row.  A lane writes four rows 4 lane + q apart by 832 bytes, which
// without the swizzle fall into 4 bank positions of a 256-byte bank row (an
// 8-16-way conflict on every feature store); with it the 16 lanes of a
// 128-bit store hit 16 distinct 16-byte slots.  The MFMA operand reads take
// 16 consecutive rows with one (r >> 4), so they stay conflict-free.
__device__ __forceinline__ int xrow_chunk(int r, int c) { return (c & ~3) | ((c & 3) ^ ((r >> 4) & 3)); }

// Block variant for the contiguous channel-major map the render writes
// (pixel stride 1, channel stride a multiple of 4, 16-byte aligned): the
// workgroup takes 256 pixels per iteration, and wave w of NWV loads channels
// [w C/NWV, (w+1) C/NWV) of all 256 with one float4 (4 pixels) per lane, so
// each channel is read as one 1 KiB run (channel-major reads in 256-byte runs
// stall at ~3.6 TB/s on MI355X, 1 KiB runs reach ~6.1 TB/s).  The waves write
// the 16-bit features into the shared pixel rows, compute their own pixels'
// SH terms, and after a barrier each wave runs the three layers on its
// 256/NWV rows as mlp_mfma32_kernel does, NJ 16-pixel N-tiles at a time.
// The next block's features are in flight during the contraction.
//  - width 32/64: 4 waves of 64 pixels, two N-tiles at a time, LDS sized at
//    launch (two workgroups per CU);
//  - width 128: the weights alone take 66 KB of LDS, so one workgroup holds a
//    CU; 8 waves of 32 pixels keep two waves on every SIMD.
template <int NT, bool kBF16, int C, int NWV, int NJ>
__global__ void __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2)))
mlp_block_kernel(const MlpParams p) {
  using S = Mlp32Shape<C, NT>;
  constexpr int K1 = S::K1, LD1 = S::LD1, LD2 = S::LD2, W = NT * 16;
  constexpr int kThreads = 64 * NWV;
  constexpr int PPW = 256 / NWV;  // pixels each wave contracts
  constexpr int NTW = PPW / 16;   // their 16-pixel N-tiles
  constexpr int CPW = C / NWV;    // channels each wave loads
  static_assert(NT % 2 == 0 && CPW % 4 == 0 && NTW % NJ == 0, "width multiple of 32, 4 channels per wave");
  static_assert(S::X + 256 * LD1 == S::TOTAL, "256 pixel rows");
  extern __shared__ uint16_t lds[];
  uint16_t* w1 = lds + S::W1;
  uint16_t* w2 = lds + S::W2;
  uint16_t* w3 = lds + S::W3;
  const uint16_t* g1 = static_cast<const uint16_t*>(p.w1);
  const uint16_t* g2 = static_cast<const uint16_t*>(p.w2);
  const uint16_t* g3 = static_cast<const uint16_t*>(p.w3);
  constexpr int Kin = C + 16;
  for (int i = threadIdx.x; i < W * LD1; i += kThreads) {
    const int r = i / LD1, k = i % LD1;
    w1[i] = k < Kin ? g1[r * Kin + k] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < W * LD2; i += kThreads) {
    const int r = i / LD2, q = i % LD2;
    w2[i] = q < W ? g2[r * W + hidden_unit(q)] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < 16 * LD2; i += kThreads) {
    const int r = i / LD2, q = i % LD2;
    w3[i] = (r < 3 && q < W) ? g3[r * W + hidden_unit(q)] : (uint16_t)0;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  uint16_t* xall = lds + S::X;              // [256 pixels][LD1], chunks swizzled by xrow_chunk
  uint16_t* xrow = xall + wid * PPW * LD1;  // this wave's PPW pixels
  if (lane < PPW)
    for (int k = Kin; k < K1; k++) xrow[lane * LD1 + 8 * xrow_chunk(wid * PPW + lane, k >> 3) + (k & 7)] = 0;

  const uint32_t N = (uint32_t)p.N;
  const uint32_t nblk = (N + 255) / 256;
  const uint32_t cs = (uint32_t)p.feat_cs;
  const float* fbase = p.feat + (size_t)(wid * CPW) * cs;  // this wave's first channel
  float4 fv[CPW];
  auto load_block = [&](uint32_t b) {
    const uint32_t n0 = b * 256 + 4 * lane;
    if (n0 + 3 < N) {
#pragma unroll
      for (int j = 0; j < CPW; j++) fv[j] = *reinterpret_cast<const float4*>(fbase + (size_t)j * cs + n0);
    } else {  // last block: clamp each pixel
      const uint32_t m0 = n0 < N ? n0 : N - 1, m1 = n0 + 1 < N ? n0 + 1 : N - 1;
      const uint32_t m2 = n0 + 2 < N ? n0 + 2 : N - 1, m3 = n0 + 3 < N ? n0 + 3 : N - 1;
#pragma unroll
      for (int j = 0; j < CPW; j++) {
        const float* c = fbase + (size_t)j * cs;
        fv[j] = make_float4(c[m0], c[m1], c[m2], c[m3]);
      }
    }
  };
  float alpha4[NTW];
#pragma unroll
  for (int j = 0; j < NTW; j++) alpha4[j] = 1.0f;
  auto load_alpha = [&](uint32_t b) {
    if (p.alpha && grp == 0) {
#pragma unroll
      for (int j = 0; j < NTW; j++) {
        const uint32_t nj = b * 256 + wid * PPW + 16 * j + col;
        alpha4[j] = p.alpha[nj < N ? nj : N - 1];
      }
    }
  };
  if (blockIdx.x < nblk) {
    load_alpha(blockIdx.x);
    load_block(blockIdx.x);
  }
  for (uint32_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    __syncthreads();  // the previous block's rows are read (and the weights written)
    // features: 4 pixel rows per lane, this wave's CPW channels, 4 channels per store
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int r = 4 * lane + q;
      uint16_t* dst = xall + r * LD1;
      uint32_t w[CPW / 2];
#pragma unroll
      for (int j = 0; j < CPW; j += 2) {
        const float v0 = q == 0 ? fv[j].x : q == 1 ? fv[j].y : q == 2 ? fv[j].z : fv[j].w;
        const float v1 = q == 0 ? fv[j + 1].x : q == 1 ? fv[j + 1].y : q == 2 ? fv[j + 1].z : fv[j + 1].w;
        w[j / 2] = pack2_16<kBF16>(v0, v1);
      }
      if constexpr (CPW % 8 == 0) {
#pragma unroll
        for (int h = 0; h < CPW / 8; h++)
          *reinterpret_cast<uint4*>(dst + 8 * xrow_chunk(r, wid * (CPW / 8) + h)) =
              make_uint4(w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]);
      } else {  // 4 channels per wave: half a chunk
        const int k0 = wid * CPW;
        *reinterpret_cast<uint2*>(dst + 8 * xrow_chunk(r, k0 >> 3) + (k0 & 7)) = make_uint2(w[0], w[1]);
      }
    }
    // SH terms of this wave's pixels
    if (lane < PPW) {
      const uint32_t n = b * 256 + wid * PPW + lane;
      float dx, dy, dz;
      pixel_dir32(p, n < N ? n : N - 1, dx, dy, dz);
      float sh[16];
      sh16(dx, dy, dz, sh);
#pragma unroll
      for (int q = 0; q < 2; q++)
        *reinterpret_cast<uint4*>(xrow + lane * LD1 + 8 * xrow_chunk(wid * PPW + lane, C / 8 + q)) =
            make_uint4(pack2_16<kBF16>(sh[8 * q + 0], sh[8 * q + 1]), pack2_16<kBF16>(sh[8 * q + 2], sh[8 * q + 3]),
                       pack2_16<kBF16>(sh[8 * q + 4], sh[8 * q + 5]), pack2_16<kBF16>(sh[8 * q + 6], sh[8 * q + 7]));
    }
    float a_out[NTW];
#pragma unroll
    for (int j = 0; j < NTW; j++) a_out[j] = alpha4[j];
    if (b + gridDim.x < nblk) {  // next block in flight during the contraction
      load_alpha(b + gridDim.x);
      load_block(b + gridDim.x);
    }
    // Every wave's channels are in the rows.  The LDS-only release/acquire
    // fences order this wave's row stores before the barrier and the other
    // waves' row reads after it (lgkmcnt 0, no wait for the block in flight);
    // a plain __syncthreads would also wait for those loads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    // NJ N-tiles at a time, so the accumulators (2 x NT x NJ x 4 floats)
    // leave room for the block in flight
#pragma unroll
    for (int h = 0; h < NTW / NJ; h++) {
      f32x4 acc1[NT][NJ];
#pragma unroll
      for (int mt = 0; mt < NT; mt++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc1[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < K1 / 32; kc++) {
        uint4 bb[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++)
          bb[j] = *reinterpret_cast<const uint4*>(xrow + (16 * (NJ * h + j) + col) * LD1 +
                                                  8 * xrow_chunk(wid * PPW + 16 * (NJ * h + j), 4 * kc + grp));
#pragma unroll
        for (int mt = 0; mt < NT; mt++) {
          const uint4 a = *reinterpret_cast<const uint4*>(w1 + (16 * mt + col) * LD1 + 32 * kc + 8 * grp);
#pragma unroll
          for (int j = 0; j < NJ; j++) acc1[mt][j] = mfma32<kBF16>(a, bb[j], acc1[mt][j]);
        }
      }
      f32x4 acc2[NT][NJ];
#pragma unroll
      for (int mt = 0; mt < NT; mt++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc2[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < NT / 2; kc++) {
        uint4 bb[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) bb[j] = relu_pack8<kBF16>(acc1[2 * kc][j], acc1[2 * kc + 1][j]);
#pragma unroll
        for (int mt = 0; mt < NT; mt++) {
          const uint4 a = *reinterpret_cast<const uint4*>(w2 + (16 * mt + col) * LD2 + 32 * kc + 8 * grp);
#pragma unroll
          for (int j = 0; j < NJ; j++) acc2[mt][j] = mfma32<kBF16>(a, bb[j], acc2[mt][j]);
        }
      }
      f32x4 acc3[NJ];
#pragma unroll
      for (int j = 0; j < NJ; j++) acc3[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < NT / 2; kc++) {
        const uint4 a = *reinterpret_cast<const uint4*>(w3 + col * LD2 + 32 * kc + 8 * grp);
#pragma unroll
        for (int j = 0; j < NJ; j++)
          acc3[j] = mfma32<kBF16>(a, relu_pack8<kBF16>(acc2[2 * kc][j], acc2[2 * kc + 1][j]), acc3[j]);
      }
      if (grp == 0) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          const uint32_t nj = b * 256 + wid * PPW + 16 * (NJ * h + j) + col;
          if (nj < N) {
#pragma unroll
            for (int o = 0; o < 3; o++)
              p.out[o * p.out_os + (int64_t)nj * p.out_ns] = finish_rgb_alpha(p, a_out[NJ * h + j], acc3[j][o], o);
          }
        }
      }
    }
  }
}

static bool mlp_block_fits(const MlpParams& p) {
  return p.feat_ns == 1 && p.feat_cs % 4 == 0 && (reinterpret_cast<uintptr_t>(p.feat) & 15u) == 0 &&
         p.N < (1ll << 31) - 256 && (uint64_t)p.feat_cs < (1ull << 31);
}

// Widths 32 and 64: 4 waves, two workgroups per CU (512 in all).  Width 128:
// 8 waves, one workgroup per CU (256 in all).
template <int NT, bool kBF16, int C>
static hipError_t launch_block(const MlpParams& p, hipStream_t s) {
  constexpr int kWaves = NT >= 8 ? 8 : 4;
  const size_t lds = sizeof(uint16_t) * (size_t)Mlp32Shape<C, NT>::TOTAL;
  const int64_t nblk = (p.N + 255) / 256;
  const int64_t cap = NT >= 8 ? 256 : 512;
  const unsigned blocks = (unsigned)(nblk < cap ? (nblk > 0 ? nblk : 1) : cap);
  hipLaunchKernelGGL((mlp_block_kernel<NT, kBF16, C, kWaves, 2>), dim3(blocks), dim3(64 * kWaves), lds, s, p);
  return hipGetLastError();
}

template <int NT, bool kBF16, int C>
static hipError_t launch_mfma32(const MlpParams& p, hipStream_t s) {
  if (mlp_block_fits(p)) return launch_block<NT, kBF16, C>(p, s);
  const size_t lds = sizeof(uint16_t) * (size_t)Mlp32Shape<C, NT>::TOTAL;
  const int64_t ntile = (p.N + 63) / 64;
  const int64_t want = (ntile + kMlp32Waves - 1) / kMlp32Waves;
  const unsigned blocks = (unsigned)(want < 1024 ? (want > 0 ? want : 1) : 1024);
  hipLaunchKernelGGL((mlp_mfma32_kernel<NT, kBF16, C>), dim3(blocks), dim3(kMlpThreads), lds, s, p);
  return hipGetLastError();
}

// float32 path on the vector ALU: one lane per pixel, weights in LDS, one
// wave per workgroup so that a small image still spreads over every CU (a
// 128x128 frame is 256 workgroups instead of 64).
constexpr int kMlpF32Threads = 64;

template <int NW>
__global__ void __launch_bounds__(kMlpF32Threads) mlp_f32_kernel(const MlpParams p) {
  extern __shared__ float wl[];
  const int C = p.C, Kin = C + 16;
  float* w1 = wl;
  float* w2 = w1 + NW * Kin;
  float* w3 = w2 + NW * NW;
  const float* g1 = static_cast<const float*>(p.w1);
  const float* g2 = static_cast<const float*>(p.w2);
  const float* g3 = static_cast<const float*>(p.w3);
  // W1 transposed to [k][j]: a feature's NW weights are one contiguous run,
  // read four at a time
  for (int i = threadIdx.x; i < NW * Kin; i += kMlpF32Threads) w1[(i % Kin) * NW + i / Kin] = g1[i];
  for (int i = threadIdx.x; i < NW * NW; i += kMlpF32Threads) w2[i] = g2[i];
  for (int i = threadIdx.x; i < 3 * NW; i += kMlpF32Threads) w3[i] = g3[i];
  __syncthreads();
  for (int64_t n = (int64_t)blockIdx.x * kMlpF32Threads + threadIdx.x; n < p.N; n += (int64_t)gridDim.x * kMlpF32Threads) {
    float dx, dy, dz;
    pixel_dir(p, n, dx, dy, dz);
    float sh[16];
    sh16(dx, dy, dz, sh);
    float h1[NW];
#pragma unroll
    for (int j = 0; j < NW; j++) h1[j] = 0.0f;
    for (int k = 0; k < C; k++) {
      const float xk = p.feat[(int64_t)k * p.feat_cs + n * p.feat_ns];
      const float4* wk = reinterpret_cast<const float4*>(w1 + k * NW);
#pragma unroll
      for (int j = 0; j < NW / 4; j++) {
        const float4 w = wk[j];
        h1[4 * j] += w.x * xk;
        h1[4 * j + 1] += w.y * xk;
        h1[4 * j + 2] += w.z * xk;
        h1[4 * j + 3] += w.w * xk;
      }
    }
#pragma unroll
    for (int s = 0; s < 16; s++) {
      const float4* wk = reinterpret_cast<const float4*>(w1 + (C + s) * NW);
#pragma unroll
      for (int j = 0; j < NW / 4; j++) {
        const float4 w = wk[j];
        h1[4 * j] += w.x * sh[s];
        h1[4 * j + 1] += w.y * sh[s];
        h1[4 * j + 2] += w.z * sh[s];
        h1[4 * j + 3] += w.w * sh[s];
      }
    }
#pragma unroll
    for (int j = 0; j < NW; j++) h1[j] = fmaxf(h1[j], 0.0f);
    float o0 = 0.f, o1 = 0.f, o2 = 0.f;
    for (int j = 0; j < NW; j++) {
      float h = 0.0f;
      const float4* wj = reinterpret_cast<const float4*>(w2 + j * NW);
#pragma unroll
      for (int k = 0; k < NW / 4; k++) {
        const float4 w = wj[k];
        h += w.x * h1[4 * k];
        h += w.y * h1[4 * k + 1];
        h += w.z * h1[4 * k + 2];
        h += w.w * h1[4 * k + 3];
      }
      h = fmaxf(h, 0.0f);
      o0 += w3[j] * h;
      o1 += w3[NW + j] * h;
      o2 += w3[2 * NW + j] * h;
    }
    p.out[0 * p.out_os + n * p.out_ns] = finish_rgb(p, n, o0, 0);
    p.out[1 * p.out_os + n * p.out_ns] = finish_rgb(p, n, o1, 1);
    p.out[2 * p.out_os + n * p.out_ns] = finish_rgb(p, n, o2, 2);
  }
}

template <int NT, bool kBF16, int KF>
static hipError_t launch_mfma_kf(const MlpParams& p, hipStream_t s) {
  const int KC1 = (p.C + 16 + 15) / 16;
  const size_t lds = sizeof(uint16_t) * ((size_t)NT * 16 * (KC1 * 16 + 4) + (size_t)NT * 16 * (NT * 16 + 4) +
                                         16 * (size_t)(NT * 16 + 4));
  const int64_t ntile = (p.N + 15) / 16;
  const int64_t want = (ntile + 3) / 4;
  const unsigned blocks = (unsigned)(want < 2048 ? (want > 0 ? want : 1) : 2048);
  hipLaunchKernelGGL((mlp_mfma_kernel<NT, kBF16, KF>), dim3(blocks), dim3(kMlpThreads), lds, s, p);
  return hipGetLastError();
}

// Feature widths that fill whole 16-channel chunks (16, 32, 64) take the
// batched-load instantiation.
template <int NT, bool kBF16>
static hipError_t launch_mfma(const MlpParams& p, hipStream_t s) {
  switch (p.C) {
    case 16: return launch_mfma_kf<NT, kBF16, 1>(p, s);
    case 32: return launch_mfma_kf<NT, kBF16, 2>(p, s);
    case 64: return launch_mfma_kf<NT, kBF16, 4>(p, s);
    default: return launch_mfma_kf<NT, kBF16, 0>(p, s);
  }
}

template <int NW>
static hipError_t launch_f32(const MlpParams& p, hipStream_t s) {
  const size_t lds = sizeof(float) * ((size_t)NW * (p.C + 16) + (size_t)NW * NW + 3 * (size_t)NW);
  const int64_t want = (p.N + kMlpF32Threads - 1) / kMlpF32Threads;
  const unsigned blocks = (unsigned)(want < 8192 ? (want > 0 ? want : 1) : 8192);
  hipLaunchKernelGGL(mlp_f32_kernel<NW>, dim3(blocks), dim3(kMlpF32Threads), lds, s, p);
  return hipGetLastError();
}

template <bool kBF16>
static hipError_t launch_mfma_width(const MlpParams& p, hipStream_t s) {
  // 64 channels at width 128 in the render's layout: the 8-wave block kernel
  if (p.width == 128 && p.C == 64 && mlp32_fits(p, p.C) && mlp_block_fits(p)) return launch_block<8, kBF16, 64>(p, s);
  // 16, 32 or 64 channels at width 32 or 64: the 16x16x32 kernel
  if ((p.width == 64 || p.width == 32) && mlp32_fits(p, p.C)) {
    const bool w64 = p.width == 64;
    switch (p.C) {
      case 16: return w64 ? launch_mfma32<4, kBF16, 16>(p, s) : launch_mfma32<2, kBF16, 16>(p, s);
      case 32: return w64 ? launch_mfma32<4, kBF16, 32>(p, s) : launch_mfma32<2, kBF16, 32>(p, s);
      case 64: return w64 ? launch_mfma32<4, kBF16, 64>(p, s) : launch_mfma32<2, kBF16, 64>(p, s);
      default: break;
    }
  }
  switch (p.width) {
    case 32: return launch_mfma<2, kBF16>(p, s);
    case 64: return launch_mfma<4, kBF16>(p, s);
    case 128: return launch_mfma<8, kBF16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_mlp(const MlpParams& p, hipStream_t s) {
  if (p.N <= 0) return hipSuccess;
  if (p.dtype == NEST_DTYPE_F32) {
    switch (p.width) {
      case 16: return launch_f32<16>(p, s);
      case 32: return launch_f32<32>(p, s);
      case 64: return launch_f32<64>(p, s);
      default: return hipErrorInvalidValue;
    }
  }
  return p.dtype == NEST_DTYPE_BF16 ? launch_mfma_width<true>(p, s) : launch_mfma_width<false>(p, s);
}

}  // namespace nest
