// Splat preprocess: projection of 2D surfels, screen AABB, tiles touched, and
// the packed 128-byte render record.
//
// Semantics: preprocessCUDA (CR/forward.cu:323-441) with compute_transmat
// (:237-290), compute_aabb (:294-320), in_frustum / quat_to_rotmat / getRect
// (CR/auxiliary.h:72-82, :190-240) and, for the colour path without
// precomputed colours, computeColorFromSH (CR/forward.cu:21-72, called at
// :417-424) -- CR = submodules/diff-surfel-rasterization/cuda_rasterizer.
//
// One lane per splat; every input is read once with 4/8/16-byte loads and the
// record is written as eight 16-byte stores (one 128-byte line per splat), so
// the render kernel can stage a splat with a single line fetch.
#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

// Real spherical-harmonic normalisations of degrees 0-3 in the basis order of
// the 3DGS colour model: C0 = 1/(2 sqrt(pi)), C1 = sqrt(3/(4 pi)),
// C2 = {sqrt(15/pi)/2, -sqrt(15/pi)/2, sqrt(5/pi)/4, -sqrt(15/pi)/2,
// sqrt(15/pi)/4}, C3 = {-sqrt(35/(2 pi))/4, sqrt(105/pi)/2, -sqrt(21/(2 pi))/4,
// sqrt(7/pi)/4, -sqrt(21/(2 pi))/4, sqrt(105/pi)/4, -sqrt(35/(2 pi))/4}.
constexpr float kShC0 = 0.28209479177387814f;
constexpr float kShC1 = 0.4886025119029199f;
constexpr float kShC2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f, -1.0925484305920792f,
                            0.5462742152960396f};
constexpr float kShC3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f, 0.3731763325901154f,
                            -0.4570457994644658f, 1.445305721320277f, -0.5900435899266435f};

// RGB of splat i from its SH coefficients (sh: M rows of 3 floats) seen from
// campos, evaluated term by term in the reference's order; + 0.5, then
// negative channels clamp to 0 and are flagged.
__device__ __forceinline__ void sh_to_rgb(int deg, const float* sh, float px, float py, float pz, const float* campos,
                                          float rgb[3], uint8_t clamped[3]) {
  float dx = px - campos[0], dy = py - campos[1], dz = pz - campos[2];
  const float len = sqrtf(dx * dx + dy * dy + dz * dz);
  dx = dx / len;
  dy = dy / len;
  dz = dz / len;
#pragma unroll
  for (int c = 0; c < 3; c++) {
    float r = kShC0 * sh[c];
    if (deg > 0) {
      const float x = dx, y = dy, z = dz;
      r = r - kShC1 * y * sh[3 + c] + kShC1 * z * sh[6 + c] - kShC1 * x * sh[9 + c];
      if (deg > 1) {
        const float xx = x * x, yy = y * y, zz = z * z;
        const float xy = x * y, yz = y * z, xz = x * z;
        r = r + kShC2[0] * xy * sh[12 + c] + kShC2[1] * yz * sh[15 + c] + kShC2[2] * (2.0f * zz - xx - yy) * sh[18 + c] +
            kShC2[3] * xz * sh[21 + c] + kShC2[4] * (xx - yy) * sh[24 + c];
        if (deg > 2) {
          r = r + kShC3[0] * y * (3.0f * xx - yy) * sh[27 + c] + kShC3[1] * xy * z * sh[30 + c] +
              kShC3[2] * y * (4.0f * zz - xx - yy) * sh[33 + c] +
              kShC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy) * sh[36 + c] +
              kShC3[4] * x * (4.0f * zz - xx - yy) * sh[39 + c] + kShC3[5] * z * (xx - yy) * sh[42 + c] +
              kShC3[6] * x * (xx - 3.0f * yy) * sh[45 + c];
        }
      }
    }
    r += 0.5f;
    clamped[c] = r < 0.0f ? 1 : 0;
    rgb[c] = r < 0.0f ? 0.0f : r;
  }
}

__global__ void __launch_bounds__(256) preprocess_kernel(const PreprocessParams p) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.P) return;

  // Defaults for culled splats (CR/forward.cu:353-354).
  p.radii[i] = 0;
  if (p.radii_user) p.radii_user[i] = 0;
  p.tiles[i] = 0;
  reinterpret_cast<uint2*>(p.rect)[i] = make_uint2(0u, 0u);
  p.depth_key[i] = 0xffffffffu;  // culled splats, which emit no pairs, go last

  const float px = p.means[3 * i + 0], py = p.means[3 * i + 1], pz = p.means[3 * i + 2];
  const float* V = p.view;
  const float vx = V[0] * px + V[4] * py + V[8] * pz + V[12];
  const float vy = V[1] * px + V[5] * py + V[9] * pz + V[13];
  const float vz = V[2] * px + V[6] * py + V[10] * pz + V[14];
  if (vz <= 0.2f) return;  // near cull, CR/auxiliary.h:205

  // quat_to_rotmat with rsqrtf -> 1/sqrtf (CR/auxiliary.h:218-240).
  const float4 q = reinterpret_cast<const float4*>(p.rots)[i];
  const float s = 1.0f / sqrtf(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  const float w = q.x * s, x = q.y * s, y = q.z * s, z = q.w * s;
  const float R00 = 1.f - 2.f * (y * y + z * z);
  const float R01 = 2.f * (x * y + w * z);
  const float R02 = 2.f * (x * z - w * y);
  const float R10 = 2.f * (x * y - w * z);
  const float R11 = 1.f - 2.f * (x * x + z * z);
  const float R12 = 2.f * (y * z + w * x);
  const float R20 = 2.f * (x * z + w * y);
  const float R21 = 2.f * (y * z - w * x);
  const float R22 = 1.f - 2.f * (x * x + y * y);
  const float2 sc = reinterpret_cast<const float2*>(p.scales)[i];
  const float s0 = p.scale_mod * sc.x, s1 = p.scale_mod * sc.y;
  const float L00 = R00 * s0, L01 = R01 * s0, L02 = R02 * s0;  // column 0 of R*S
  const float L10 = R10 * s1, L11 = R11 * s1, L12 = R12 * s1;  // column 1

  // T = transpose(splat2world) * world2ndc * ndc2pix (CR/forward.cu:255-274)
  const float* A = p.proj;
  float M[3][4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    M[0][c] = L00 * A[c] + L01 * A[4 + c] + L02 * A[8 + c];
    M[1][c] = L10 * A[c] + L11 * A[4 + c] + L12 * A[8 + c];
    M[2][c] = px * A[c] + py * A[4 + c] + pz * A[8 + c] + A[12 + c];
  }
  const float hw = (float)p.W / 2.0f, hh = (float)p.H / 2.0f;
  const float cw = (float)(p.W - 1) / 2.0f, ch = (float)(p.H - 1) / 2.0f;
  float Tu[3], Tv[3], Tw[3];
#pragma unroll
  for (int r = 0; r < 3; r++) {
    Tu[r] = M[r][0] * hw + M[r][3] * cw;
    Tv[r] = M[r][1] * hh + M[r][3] * ch;
    Tw[r] = M[r][3];
  }

  // View-space normal of the splat's third axis, normalised, facing the camera.
  float nx = V[0] * R20 + V[4] * R21 + V[8] * R22;
  float ny = V[1] * R20 + V[5] * R21 + V[9] * R22;
  float nz = V[2] * R20 + V[6] * R21 + V[10] * R22;
  const float nlen = sqrtf(nx * nx + ny * ny + nz * nz);
  if (nlen > 1e-7f) { nx = nx / nlen; ny = ny / nlen; nz = nz / nlen; }
  const float cosv = -(vx * nx + vy * ny + vz * nz);
  if (cosv == 0.0f) return;
  const float mul = cosv > 0.0f ? 1.0f : -1.0f;
  nx = mul * nx; ny = mul * ny; nz = mul * nz;

  // compute_aabb with cutoff 4.
  const float cut2 = 16.0f;
  const float d = cut2 * (Tw[0] * Tw[0]) + cut2 * (Tw[1] * Tw[1]) + -1.0f * (Tw[2] * Tw[2]);
  if (d == 0.0f) return;
  const float invd = 1.0f / d;
  const float f0 = invd * cut2, f1 = invd * cut2, f2 = invd * -1.0f;
  const float pimx = f0 * (Tu[0] * Tw[0]) + f1 * (Tu[1] * Tw[1]) + f2 * (Tu[2] * Tw[2]);
  const float pimy = f0 * (Tv[0] * Tw[0]) + f1 * (Tv[1] * Tw[1]) + f2 * (Tv[2] * Tw[2]);
  const float h0x = pimx * pimx - (f0 * (Tu[0] * Tu[0]) + f1 * (Tu[1] * Tu[1]) + f2 * (Tu[2] * Tu[2]));
  const float h0y = pimy * pimy - (f0 * (Tv[0] * Tv[0]) + f1 * (Tv[1] * Tv[1]) + f2 * (Tv[2] * Tv[2]));
  const float ex = sqrtf(fmaxf(1e-4f, h0x));
  const float ey = sqrtf(fmaxf(1e-4f, h0y));
  const float radius = ceilf(fmaxf(fmaxf(ex, ey), 4.0f * 0.707106f));
  const int ir = f2i_sat(radius);

  uint32_t x0, y0, x1, y1;
  tile_rect(pimx, pimy, ir, p.gx, p.gy, x0, y0, x1, y1);
  const uint32_t area = (x1 - x0) * (y1 - y0);
  if (area == 0) return;

  const float opacity = p.opac[i];
  p.depth[i] = vz;
  p.radii[i] = ir;
  if (p.radii_user) p.radii_user[i] = ir;
  reinterpret_cast<float2*>(p.xy)[i] = make_float2(pimx, pimy);
  p.tiles[i] = area;
  reinterpret_cast<uint2*>(p.rect)[i] = make_uint2(x0 | y0 << 16, x1 | y1 << 16);
  p.depth_key[i] = __float_as_uint(vz);  // vz > 0.2: the bit order is the float order
  if (p.shs) {
    float rgb[3];
    uint8_t cl[3];
    sh_to_rgb(p.sh_degree, p.shs + (size_t)i * p.sh_coeffs * 3, px, py, pz, p.campos, rgb, cl);
#pragma unroll
    for (int c = 0; c < 3; c++) {
      p.rgb[3 * (size_t)i + c] = rgb[c];
      p.clamped[3 * (size_t)i + c] = cl[c];
    }
  }

  uint32_t ap = 0xffffffffu;
  if (p.ap_level) ap = f2u_sat(floorf(p.ap_level[i]));
  float su0 = 0.f, su1 = 0.f, su2 = 0.f, sv0 = 0.f, sv1 = 0.f, sv2 = 0.f, pk0 = 0.f, pk1 = 0.f, pk2 = 0.f;
  if (p.homotrans) {
    const float4* Hm = reinterpret_cast<const float4*>(p.homotrans) + 4 * (size_t)i;
    const float4 r0 = Hm[0], r1 = Hm[1], r2 = Hm[2];
    su0 = r0.x; su1 = r1.x; su2 = r2.x;
    sv0 = r0.y; sv1 = r1.y; sv2 = r2.y;
    pk0 = r0.w; pk1 = r1.w; pk2 = r2.w;
  }
  // Rejection bounds for the render loop.  A pair is rejected by the alpha
  // test (alpha < 1/255) whenever rho = min(rho3d, rho2d) > 2 ln(255 o); with
  // the beta activation G' = (1+b) G / (1+b G) the bound is
  // 2 ln(255 o (1+b) - b) (G' = 1/(255 o) solved for G).  The cut below adds
  // a relative 1e-6 for the expf/rounding error and 1e-4 absolute, so any
  // pair the render skips with it is one the exact test rejects.  The acceptance region {rho3d <= cut} U {rho2d <= cut} is
  // bounded by the bbox of the projected disk |s|^2 <= cut (the conic bbox of
  // CR/forward.cu:294-320 at cutoff^2 = cut, valid when the whole disk lies in
  // front of the camera: cut*(Tw0^2+Tw1^2) < Tw2^2) and the disk of radius
  // sqrt(cut/2) around xy, widened by one pixel.
  // The other kernels (CR/forward.cu:864-900) bound rho the same way: the
  // beta kernel accepts only rho < 1 and alpha >= 1/255 needs
  // rho <= 1 - (255 o)^(-1/shape); the flex kernel is the Gaussian with the
  // splat's own beta; the general kernel needs rho <= (2 ln(255 o))^(2/shape).
  // Their powers are not correctly rounded (powf_ref), hence the wider
  // relative margins.  A parameter without a finite bound (NaN, or a
  // non-positive exponent of the general kernel) takes the exact path.
  float cut = -1.0f;
  float bx0 = 1.0f, bx1 = -1.0f, by0 = 1.0f, by1 = -1.0f;  // empty: never accepted
  const float shape = p.kernel_type != 0 ? p.shapes[i] : 0.0f;
  const double sh = (double)shape;
  double bb = p.kernel_type == 0 && p.beta > 0.0f ? (double)p.beta : 0.0;
  if (p.kernel_type == 2) bb = shape > 0.0f ? sh : 0.0;
  const double xo = 255.0 * (double)opacity * (1.0 + bb) - bb;
  const bool finite_shape = p.kernel_type == 0 || p.kernel_type == 2 || (shape == shape && (p.kernel_type != 3 || shape > 0.0f));
  if (opacity > 0.0f && xo > 0.0 && finite_shape) {
    double c = 2.0 * log(xo * (1.0 + 1e-6)) + 1e-4;
    if (p.kernel_type == 1) {
      // rho < 1 always; alpha >= 1/255 bounds it further for a positive shape
      const double o255 = 255.0 * (double)opacity;
      c = 1.0;
      if (shape > 0.0f && o255 > 1.0) c = fmin(1.0, 1.0 - pow(o255, -1.0 / sh) + 1e-3);
      if (o255 <= 1.0 && shape > 0.0f) c = -1.0;  // base^shape <= 1: never 1/255
    } else if (p.kernel_type == 3) {
      const double c0 = 2.0 * log(255.0 * (double)opacity) * (1.0 + 1e-4) + 1e-4;
      c = c0 > 0.0 ? pow(c0, 2.0 / sh) * (1.0 + 1e-3) + 1e-3 : -1.0;
    }
    if (c >= 0.0) {
      cut = (float)c;
      const double rd = sqrt(c * 0.5) + 1.0;
      bx0 = (float)(pimx - rd); bx1 = (float)(pimx + rd);
      by0 = (float)(pimy - rd); by1 = (float)(pimy + rd);
      const double w0 = Tw[0], w1 = Tw[1], w2 = Tw[2];
      const double dd = c * (w0 * w0 + w1 * w1) - w2 * w2;
      if (dd < 0.0 && w2 > 0.0) {
        const double f0 = c / dd, f2 = -1.0 / dd;
        const double ex_c = f0 * (Tu[0] * w0) + f0 * (Tu[1] * w1) + f2 * (Tu[2] * w2);
        const double ey_c = f0 * (Tv[0] * w0) + f0 * (Tv[1] * w1) + f2 * (Tv[2] * w2);
        const double hx2 = ex_c * ex_c - (f0 * ((double)Tu[0] * Tu[0]) + f0 * ((double)Tu[1] * Tu[1]) + f2 * ((double)Tu[2] * Tu[2]));
        const double hy2 = ey_c * ey_c - (f0 * ((double)Tv[0] * Tv[0]) + f0 * ((double)Tv[1] * Tv[1]) + f2 * ((double)Tv[2] * Tv[2]));
        const double hx = sqrt(hx2 > 0.0 ? hx2 : 0.0) + 1.0, hy = sqrt(hy2 > 0.0 ? hy2 : 0.0) + 1.0;
        bx0 = (float)fmin((double)bx0, ex_c - hx); bx1 = (float)fmax((double)bx1, ex_c + hx);
        by0 = (float)fmin((double)by0, ey_c - hy); by1 = (float)fmax((double)by1, ey_c + hy);
      } else {
        bx0 = -3.0e38f; bx1 = 3.0e38f; by0 = -3.0e38f; by1 = 3.0e38f;  // unbounded image: never cull
      }
    }
  } else if (!(opacity <= 0.0f)) {
    // NaN opacity, a parameter without a bound, or a beta activation that
    // keeps every alpha below 1/255: always the exact path
    cut = __int_as_float(0x7fc00000);
    bx0 = -3.0e38f; bx1 = 3.0e38f; by0 = -3.0e38f; by1 = 3.0e38f;
  }
  float4* rec = reinterpret_cast<float4*>(p.records) + 8 * (size_t)i;
  rec[0] = make_float4(Tu[0], Tu[1], Tu[2], Tv[0]);
  rec[1] = make_float4(Tv[1], Tv[2], Tw[0], Tw[1]);
  rec[2] = make_float4(Tw[2], pimx, pimy, opacity);
  rec[3] = make_float4(nx, ny, nz, __uint_as_float(ap));
  rec[4] = make_float4(su0, su1, su2, sv0);
  rec[5] = make_float4(sv1, sv2, pk0, pk1);
  rec[6] = make_float4(pk2, cut, shape, vz);
  rec[7] = make_float4(bx0, bx1, by0, by1);
}

hipError_t launch_preprocess(const PreprocessParams& p, hipStream_t s) {
  if (p.P <= 0) return hipSuccess;
  const int blocks = (p.P + 255) / 256;
  hipLaunchKernelGGL(preprocess_kernel, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

// checkFrustum / in_frustum (CR/rasterizer_impl.cu:54-66, CR/auxiliary.h:
// 190-215): only the near test p_view.z > 0.2 decides; the projected point the
// reference also computes is unused there.
struct ViewMatrix {
  float m[16];
};

__global__ void __launch_bounds__(256) mark_visible_kernel(int P, const float* __restrict__ means, const ViewMatrix V,
                                                           uint8_t* __restrict__ present) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P) return;
  const float px = means[3 * i + 0], py = means[3 * i + 1], pz = means[3 * i + 2];
  const float vz = V.m[2] * px + V.m[6] * py + V.m[10] * pz + V.m[14];
  present[i] = vz <= 0.2f ? 0 : 1;
}

hipError_t launch_mark_visible(int P, const float* means, const float view[16], uint8_t* present, hipStream_t s) {
  if (P <= 0) return hipSuccess;
  ViewMatrix V;
  for (int k = 0; k < 16; k++) V.m[k] = view[k];
  hipLaunchKernelGGL(mark_visible_kernel, dim3((P + 255) / 256), dim3(256), 0, s, P, means, V, present);
  return hipGetLastError();
}

// get_homotrans (scene/gaussian_model.py:312-317) = build_H(build_rotation(r),
// s, xyz) of utils/general_utils.py:78-113: the quaternion is normalised with
// sqrt(((r0 r0 + r1 r1) + r2 r2) + r3 r3) and a division, R is built with the
// reference's expressions, and H = [[R * (sx, sy, 0) by column, xyz],
// [0, 0, 0, 1]] row-major; every operation is one float32 rounding in the
// order the torch expressions evaluate, so the result equals the reference's
// elementwise kernels bit for bit (column 2 is 0 * R, -0 where R < 0).
__global__ void __launch_bounds__(256) homotrans_kernel(int64_t P, const float4* __restrict__ rots,
                                                        const float2* __restrict__ scales,
                                                        const float* __restrict__ means, float4* __restrict__ H) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P) return;
  const float4 q = rots[i];
  const float norm = sqrtf(((q.x * q.x + q.y * q.y) + q.z * q.z) + q.w * q.w);
  const float r = q.x / norm, x = q.y / norm, y = q.z / norm, z = q.w / norm;
  const float R00 = 1.0f - 2.0f * (y * y + z * z), R01 = 2.0f * (x * y - r * z), R02 = 2.0f * (x * z + r * y);
  const float R10 = 2.0f * (x * y + r * z), R11 = 1.0f - 2.0f * (x * x + z * z), R12 = 2.0f * (y * z - r * x);
  const float R20 = 2.0f * (x * z - r * y), R21 = 2.0f * (y * z + r * x), R22 = 1.0f - 2.0f * (x * x + y * y);
  const float2 s = scales[i];
  const float m0 = means[3 * i], m1 = means[3 * i + 1], m2 = means[3 * i + 2];
  float4* h = H + 4 * i;
  h[0] = make_float4(s.x * R00, s.y * R01, 0.0f * R02, m0);
  h[1] = make_float4(s.x * R10, s.y * R11, 0.0f * R12, m1);
  h[2] = make_float4(s.x * R20, s.y * R21, 0.0f * R22, m2);
  h[3] = make_float4(0.0f, 0.0f, 0.0f, 1.0f);
}

hipError_t launch_build_homotrans(int64_t P, const float* rots, const float* scales, const float* means, float* H,
                                  hipStream_t s) {
  if (P <= 0) return hipSuccess;
  hipLaunchKernelGGL(homotrans_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, s, P,
                     reinterpret_cast<const float4*>(rots), reinterpret_cast<const float2*>(scales), means,
                     reinterpret_cast<float4*>(H));
  return hipGetLastError();
}

}  // namespace nest
