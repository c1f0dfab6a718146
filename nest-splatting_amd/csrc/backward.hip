// Backward pass (training) of the render, mode 0 with the Gaussian kernel,
// of preprocess, and of the standalone GridEncoder.
//
// Semantics: renderCUDAsurfelBackward of
// submodules/diff-surfel-rasterization/cuda_rasterizer/backward.cu:445-2049
// (mode 0, kernel_type 0), query_feature<true> (hashgrid.h:53-299),
// compute_transmat_aabb / preprocessCUDA / computeColorFromSH backward
// (backward.cu:20-140, :2056-2274), kernel_grid_backward and
// kernel_input_backward with the forward's dy_dx (gridencoder/src/
// gridencoder.cu:196-366).
//
// Layout of the render backward: one 256-thread workgroup per 16x16 tile, one
// lane per pixel, the tile's splats walked back to front in LDS-staged
// batches of the forward's packed records.  With a grid, a wave splits each
// batch into segments: a geometry pass queues the segment's hits, the queued
// hits are spread one per lane for the grid work (table gathers, the
// features' dot product with dL/dpixel, dL/dxyz, the table-gradient scatter),
// and a third pass runs the blending recursion over the splats that hit the
// wave.  Two restructurings against the reference, both the same sums in
// another order:
//  - the reference keeps three C-long arrays per pixel (accum_rec,
//    last_color, dL_dpixel).  The back-to-front blend accum_rec =
//    a*last + (1-a)*accum_rec is linear with the same coefficients for every
//    channel, and only its dot product with dL_dpixel enters dL/dalpha, so a
//    pixel carries two scalars (the blend's and the last colour's dot
//    products with dL_dpixel) and reads its dL_dpixel values from memory
//    where a level needs them (cache-resident, coalesced across the wave);
//    the |grad| sum of a hit is w * sum |dL_dpixel|, summed once per pixel;
//  - every lane of a wave visits the same staged splat at the same time, so
//    the per-splat gradients (transmat, homotrans, mean2D, normal, opacity,
//    |grad| sum, colours) are summed over the wave with cross-lane shuffles
//    and added with one atomic per wave instead of one per pixel.
// Table gradients are hardware float atomics (global_atomic_add_f32) at
// every corner, as in the reference, merged per cell across the wave first.
// Their cost is one request per (instruction, 64-byte segment) and, on
// MI355X, a fixed share of the texture path per instruction however few
// lanes it carries, so the scatter below stages the cells' sums in LDS and
// adds them 64 consecutive values per instruction (whole entries).
#include <hip/hip_fp16.h>

#include "hashgrid.h"
#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

namespace {

constexpr int kBwdThreads = 256;
constexpr int kBwdChunks = 7;  // record chunks 0-6: T, xy, opacity, normal, ap, homotrans columns

// Cross-lane sums on the VALU (no LDS round trips): v_permlane32_swap /
// v_permlane16_swap exchange lane halves (bits 5 and 4 of the lane index),
// DPP row operations the rest.  halve<bit>(lo, hi) is one recursive-halving
// step: a lane whose index has the bit clear returns lo + its partner's lo,
// one with the bit set hi + its partner's hi, the partner differing in that
// bit (for bit 2 the partner is lane ^ 7, which leaves the bits above alone).
// The swap builtins return (a with its upper half [row] replaced by b's lower
// one, b with its lower half replaced by a's upper one), so the pair to sum
// is the two results.
constexpr int kDppRor8 = 0x128;        // row_ror:8, lane ^ 8 within a row
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror, lane ^ 7
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]

template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float halve(int bit, float lo, float hi) {
  if (bit == 5) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if (bit == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  const bool up = ((threadIdx.x >> bit) & 1u) != 0u;
  const float send = up ? lo : hi, keep = up ? hi : lo;
  float got;
  if (bit == 3)
    got = dpp_f<kDppRor8>(send);
  else if (bit == 2)
    got = dpp_f<kDppHalfMirror>(send);
  else if (bit == 1)
    got = dpp_f<kDppQuadXor2>(send);
  else
    got = dpp_f<kDppQuadXor1>(send);
  return keep + got;
}

// Sum over the 64 lanes, in every lane.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int b = 5; b >= 0; b--) v = halve(b, v, v);
  return v;
}

__device__ __forceinline__ void atomic_add(float* p, float v) { unsafeAtomicAdd(p, v); }

// Staging area of the table-gradient atomics: 256 dwords of LDS per wave,
// kSlots slots of NV = 8F summed values (a cell's corner values, corner-major)
// followed by the slots' 8 entry indices.  A flush adds nb slots with packed
// atomics: lane l of instruction r adds value 64r + l, so an instruction
// carries 64 consecutive values (for F = 4 sixteen whole 16-byte entries).
template <int F>
struct StageLayout {
  static constexpr int NV = 8 * F;
  static constexpr uint32_t kSlots = 256 / (NV + 8);
  static constexpr uint32_t kIdx = kSlots * NV;  // first index dword
};

template <int F>
__device__ __forceinline__ void stage_flush(const uint32_t* st, uint32_t nb, float* dl) {
  constexpr int NV = 8 * F;
  constexpr uint32_t kIdx = StageLayout<F>::kIdx;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t nval = nb * NV;
  for (uint32_t f0 = 0; f0 < nval; f0 += 64u) {
    const uint32_t f = f0 + lane;
    if (f < nval) {
      const float val = __uint_as_float(st[f]);
      const uint32_t h = f / NV, v = f % NV;
      const uint32_t e = st[kIdx + h * 8u + v / F];
      if (val != 0.0f) atomic_add(dl + (size_t)e * F + (v % F), val);
    }
  }
}

constexpr uint32_t kSmallCell = 8;  // cells of up to this many lanes are summed by pointer jumping

// Table gradient of one level for the wave (uniform control flow): lanes
// whose hits fall in the same cell (same g) share all eight corner entries.
// The cells are taken one at a time (the lowest remaining lane's cell and
// every lane sharing it).  A cell of more than kSmallCell lanes has its 8F
// values summed over its lanes with recursive-halving reduce-scatters, 16
// values at a time (after one, lane l holds the sum of value l / 4 of the
// chunk), written straight to a staging slot; the smaller cells are summed all
// at once after the search by pointer jumping along each cell's lanes, into
// the cell's lowest lane, which then writes a slot as a lane alone in its cell
// does.  Full sets of slots are added with packed atomics.  At coarse levels a wave's 64 hits
// (neighbouring pixels and splats adjacent in depth) are a few cells, which is
// where the per-lane atomics of the reference pile onto the same addresses; at
// fine levels a cell holds a few lanes.
template <int F>
__device__ __forceinline__ void scatter_level(bool on, const uint32_t gc[3], const uint32_t idx[8], float* cv,
                                              float* dl, uint32_t* st) {
  constexpr int NV = 8 * F;
  constexpr uint32_t kSlots = StageLayout<F>::kSlots;
  constexpr uint32_t kIdx = StageLayout<F>::kIdx;
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t rem = __ballot(on);
  uint64_t issue = 0ull;  // lanes holding a small cell's sum (or alone in their cell)
  // next lane of the lane's small cell as a byte address for ds_bpermute;
  // bit 31 set: the lane is the last of its cell (or in no small cell)
  uint32_t succ = 0x80000000u | (lane << 2);
  uint32_t small_max = 1u;
  uint32_t nb = 0u;  // staging slots in use
  while (rem != 0ull) {
    const int ld = __ffsll((long long)rem) - 1;
    const uint32_t k0 = __builtin_amdgcn_readlane(gc[0], ld), k1 = __builtin_amdgcn_readlane(gc[1], ld),
                   k2 = __builtin_amdgcn_readlane(gc[2], ld);
    const uint64_t m = __ballot(gc[0] == k0) & __ballot(gc[1] == k1) & __ballot(gc[2] == k2) & rem;
    rem &= ~m;
    const uint32_t n = (uint32_t)__popcll(m);
    if (n <= kSmallCell) {
      issue |= m & (~m + 1ull);
      if (n > 1u) {
        const uint64_t after = m & ~((2ull << lane) - 1ull);
        if (((m >> lane) & 1ull) != 0ull && after != 0ull) succ = (uint32_t)(__ffsll((long long)after) - 1) << 2;
        small_max = n > small_max ? n : small_max;
      }
      continue;
    }
    const bool mem = ((m >> lane) & 1ull) != 0ull;
    if (nb == kSlots) {
      stage_flush<F>(st, nb, dl);
      nb = 0u;
    }
    // reduce-scatter in chunks of kCh values (fewer live registers)
    constexpr int kCh = NV < 16 ? NV : 16;
    constexpr int kRepC = 64 / kCh;
#pragma unroll
    for (int c = 0; c < NV / kCh; c++) {
      float v[kCh];
#pragma unroll
      for (int i = 0; i < kCh; i++) v[i] = mem ? cv[c * kCh + i] : 0.0f;
      int vi = 0;
#pragma unroll
      for (int s = 0; (kCh >> (s + 1)) >= 1; s++) {
        const int h = kCh >> (s + 1);
        const int bit = 5 - s;
#pragma unroll
        for (int i = 0; i < h; i++) v[i] = halve(bit, v[i], v[i + h]);
        if (((lane >> bit) & 1u) != 0u) vi += h;
      }
      // lanes differing only in the bits below hold the same value index
#pragma unroll
      for (int bit = 0; (1 << bit) < kRepC; bit++) v[0] = halve(bit, v[0], v[0]);
      if ((lane % kRepC) == 0u) st[nb * NV + (uint32_t)(c * kCh + vi)] = __float_as_uint(v[0]);
      __builtin_amdgcn_sched_barrier(0);
    }
    uint32_t e = __builtin_amdgcn_readlane(idx[0], ld);
#pragma unroll
    for (int kk = 1; kk < 8; kk++) {
      const uint32_t ek = __builtin_amdgcn_readlane(idx[kk], ld);
      e = (lane == (uint32_t)kk) ? ek : e;
    }
    if (lane < 8u) st[kIdx + nb * 8u + lane] = e;
    nb++;
  }
  // small cells: pointer jumping, after which a cell's lowest lane holds the
  // sum over the cell's lanes
  for (uint32_t span = 1u; span < small_max; span <<= 1) {
    const bool has = (succ & 0x80000000u) == 0u;
    const int addr = (int)(succ & 0xFFu);
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const float got = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(cv[i])));
      if (has) cv[i] += got;
      if ((i & 7) == 7) __builtin_amdgcn_sched_barrier(0);
    }
    if (span * 2u < small_max) succ = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)succ);
  }
  const uint32_t n_iss = (uint32_t)__popcll(issue);
  const uint32_t rank = (uint32_t)__popcll(issue & ((1ull << lane) - 1ull));
  const bool me = ((issue >> lane) & 1ull) != 0ull;
  for (uint32_t done = 0; done < n_iss;) {
    if (nb == kSlots) {
      stage_flush<F>(st, nb, dl);
      nb = 0u;
    }
    const uint32_t take = min(kSlots - nb, n_iss - done);
    if (me && rank >= done && rank < done + take) {
      const uint32_t h = nb + rank - done;
      float4* sv = reinterpret_cast<float4*>(st + h * NV);
#pragma unroll
      for (int i = 0; i < NV / 4; i++) sv[i] = make_float4(cv[4 * i], cv[4 * i + 1], cv[4 * i + 2], cv[4 * i + 3]);
      uint4* si = reinterpret_cast<uint4*>(st + kIdx + h * 8u);
      si[0] = make_uint4(idx[0], idx[1], idx[2], idx[3]);
      si[1] = make_uint4(idx[4], idx[5], idx[6], idx[7]);
    }
    nb += take;
    done += take;
  }
  if (nb > 0u) stage_flush<F>(st, nb, dl);
}

// query_feature<true> for the wave's hits at grid coordinates u (lanes with
// lane_levels 0 take part with nothing): recomputes the features' projection
// dot = sum_ch feat[ch] * dpix[ch], adds w_corner * w * dpix to the table at
// every corner of every level below lane_levels, and returns dL/dxyz
// (hashgrid.h:213-299; grad_scale of :66-97).
template <int F>
__device__ __forceinline__ void hash_backward_wave(const GridParams& g, nest_i32x4 rsrc, const float u[3],
                                                   float grad_scale, uint32_t lane_levels, float w,
                                                   const float* dpix, size_t HW, float* dtable, uint32_t* st,
                                                   float& dot, float dxyz[3]) {
  dot = 0.0f;
  dxyz[0] = dxyz[1] = dxyz[2] = 0.0f;
  const LevelTable& lv = g.lv;
  for (int l = 0; l < (int)g.L; l++) {
    const bool on = (uint32_t)l < lane_levels;
    if (__ballot(on) == 0ull) break;  // levels are a prefix per lane
    const float scale = lv.scale[l];
    float cv[8 * F];
#pragma unroll
    for (int i = 0; i < 8 * F; i++) cv[i] = 0.0f;
    uint32_t gc[3] = {0u, 0u, 0u};
    LevelCorners cn;
#pragma unroll
    for (int k = 0; k < 8; k++) cn.idx[k] = 0u;
    if (on) {
      float pos[3], der[3];
#pragma unroll
      for (int d = 0; d < 3; d++) {
        const float x = u[d] * scale + g.pos_offset;
        gc[d] = f2u_sat(x);
        pos[d] = x - (float)gc[d];
        if (g.interp == 1) {
          der[d] = 6.0f * pos[d] * (1.0f - pos[d]);
          pos[d] = pos[d] * pos[d] * (3.0f - 2.0f * pos[d]);
        } else {
          der[d] = 1.0f;
        }
      }
      level_corners<F, false>(lv, l, g.pos_offset, 0u, u, cn);  // indices of the same cell
      cn.wx[0] = 1 - pos[0]; cn.wx[1] = pos[0];
      cn.wy[0] = 1 - pos[1]; cn.wy[1] = pos[1];
      cn.wz[0] = 1 - pos[2]; cn.wz[1] = pos[2];
      float vals[8][F];
      corners_load<F, false>(rsrc, cn, vals);
      float dp[F], gf[F], feat[F];
#pragma unroll
      for (int f = 0; f < F; f++) {
        dp[f] = dpix[(size_t)(l * F + f) * HW];
        gf[f] = w * dp[f];
        feat[f] = 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float wk = (1.0f * cn.wx[k & 1]) * cn.wy[(k >> 1) & 1] * cn.wz[k >> 2];
#pragma unroll
        for (int f = 0; f < F; f++) {
          feat[f] = fmaf(wk, vals[k][f], feat[f]);
          cv[k * F + f] = wk * gf[f];
        }
      }
#pragma unroll
      for (int f = 0; f < F; f++) dot += feat[f] * dp[f];
      // dy/dxyz: corner pairs along each axis (hashgrid.h:241-276)
#pragma unroll
      for (int gd = 0; gd < 3; gd++) {
        float rg[F];
#pragma unroll
        for (int f = 0; f < F; f++) rg[f] = 0.0f;
#pragma unroll
        for (int idx = 0; idx < 4; idx++) {
          float wgt = scale * grad_scale;
          int kl = 0;
#pragma unroll
          for (int nd = 0; nd < 2; nd++) {
            const int d = (nd >= gd) ? nd + 1 : nd;
            const int bit = (idx >> nd) & 1;
            wgt *= bit ? pos[d] : 1 - pos[d];
            kl |= bit << d;
          }
          const int kr = kl | (1 << gd);
#pragma unroll
          for (int f = 0; f < F; f++) rg[f] += wgt * (vals[kr][f] - vals[kl][f]) * der[gd];
        }
#pragma unroll
        for (int f = 0; f < F; f++) dxyz[gd] += gf[f] * rg[f];
      }
    }
    scatter_level<F>(on, gc, cn.idx, cv, dtable + (size_t)lv.base[l] * F, st);
  }
}

// Grid coordinate of xyz and the scalar grad_scale (hashgrid.h:66-97);
// returns false when the point is outside the grid (no features, no gradient).
__device__ __forceinline__ bool grid_coord_bwd(const GridParams& g, const float xyz[3], float u[3],
                                               float& grad_scale) {
  if (!g.contract) {
#pragma unroll
    for (int d = 0; d < 3; d++) u[d] = (xyz[d] - g.vmin) * g.inv_size;
    grad_scale = g.inv_size;
    return !(u[0] < 0 || u[0] > 1 || u[1] < 0 || u[1] > 1 || u[2] < 0 || u[2] > 1);
  }
#pragma unroll
  for (int d = 0; d < 3; d++) u[d] = (xyz[d] - g.vmid) * g.inv_size;
  const float nrm = sqrtf(u[0] * u[0] + u[1] * u[1] + u[2] * u[2]);
  const float inv_nrm = 1.0f / nrm;
  const float st = (nrm <= 1.0f) ? 1.0f : (2.0f - inv_nrm) * inv_nrm;
#pragma unroll
  for (int d = 0; d < 3; d++) {
    u[d] = st * u[d];
    u[d] = (u[d] + 2.0f) * 0.25f;
  }
  grad_scale = g.inv_size * st * 0.25f;
  return true;
}

// Per-pixel inputs and back-to-front state of the render backward
// (backward.cu:1597-1700): the pixel's output gradients, the forward's final
// T, depth sums and contributor counts, and the blending recursion (the
// colour blend as its two dot products with dL/dpixel).
struct BwdPixel {
  bool inside;
  float pxf, pyf;
  const float* dpix;  // channel c at dpix[c * HW]
  float sum_abs;
  float dL_ddepth, dL_daccum, dn2[3], dL_dmedian, dL_dreg;
  uint32_t last_contributor;
  int median_contributor;
  float final_D, final_D2, final_A;
  float T;
  float acc_dot, last_dot;  // accum_rec . dpix, last_color . dpix
  float last_depth, last_normal[3];
  float accum_depth_rec, accum_alpha_rec, accum_normal_rec[3];
  float last_dL_dT, last_alpha;
};

// Pixel (x0 + t % 16, y0 + t / 16) of thread t of the tile's workgroup.
__device__ __forceinline__ void bwd_pixel_init(const RenderBwdParams& p, uint32_t tile, BwdPixel& px) {
  const uint32_t tx = tile % p.gx, ty = tile / p.gx;
  const uint32_t x = tx * kTile + (threadIdx.x & 15u);
  const uint32_t y = ty * kTile + (threadIdx.x >> 4);
  const bool inside = x < (uint32_t)p.W && y < (uint32_t)p.H;
  const size_t HW = (size_t)p.W * p.H;
  const size_t pid = inside ? (size_t)y * p.W + x : 0;
  px.inside = inside;
  px.pxf = (float)x;
  px.pyf = (float)y;
  px.dpix = p.dL_dpix + pid;
  px.sum_abs = 0.0f;
  if (inside)
    for (int c = 0; c < p.C; c++) px.sum_abs += fabsf(px.dpix[(size_t)c * HW]);
  const float* dO = p.dL_dothers;
  px.dL_ddepth = inside ? dO[pid] : 0.0f;
  px.dL_daccum = inside ? dO[HW + pid] : 0.0f;
  px.dn2[0] = inside ? dO[2 * HW + pid] : 0.0f;
  px.dn2[1] = inside ? dO[3 * HW + pid] : 0.0f;
  px.dn2[2] = inside ? dO[4 * HW + pid] : 0.0f;
  px.dL_dmedian = inside ? dO[5 * HW + pid] : 0.0f;
  px.dL_dreg = inside ? dO[6 * HW + pid] : 0.0f;
  const float T_final = inside ? p.final_T[pid] : 0.0f;
  px.T = T_final;
  px.last_contributor = inside ? p.n_contrib[pid] : 0u;
  px.median_contributor = inside ? (int)p.n_contrib[pid + HW] : 0;
  px.final_D = inside ? p.final_T[pid + HW] : 0.0f;
  px.final_D2 = inside ? p.final_T[pid + 2 * HW] : 0.0f;
  px.final_A = 1 - T_final;
  px.acc_dot = px.last_dot = 0.0f;
  px.last_depth = 0.0f;
  px.accum_depth_rec = px.accum_alpha_rec = 0.0f;
#pragma unroll
  for (int c = 0; c < 3; c++) px.last_normal[c] = px.accum_normal_rec[c] = 0.0f;
  px.last_dL_dT = px.last_alpha = 0.0f;
}

// Ray/splat intersection of one staged record at the pixel.
struct BwdHit {
  float k[3], l[3], pp[3];
  float s[2], d[2];
  float c_d, G, demon, alpha;
  // kernel types 1-3: dG/ds = pf * s (3D; 2 pf * d in 2D), dL/dG scale gsc, dG/dshape gs
  float pf, gsc, gs;
  bool use3d;
};

// G of kernel types 1-3 and the factors of its gradients, as
// CR/backward.cu:764-800 and :1864-1909, :1958-2032 write them: the beta
// kernel's position factor is -shape G / base (half the derivative of
// (1 - rho)^shape in s, which the reference keeps), the flex kernel's the raw
// Gaussian's with dL/dG scaled by (1 + b) / demon^2, and no shape gradient
// at b <= 0.  False for a pair the kernel rejects.
__device__ __forceinline__ bool bwd_kernel_g(int kt, float rho, float shape, BwdHit& h) {
  h.gsc = 1.0f;
  h.gs = 0.0f;
  if (kt == 1) {
    if (rho >= 1.0f) return false;
    const float base = 1.0f - rho;
    h.G = powf_ref(base, shape);
    h.pf = base > 1e-7f ? -shape * h.G / base : 0.0f;
    if (base > 1e-7f) h.gs = h.G * logf_ref(base);
    return true;
  }
  if (kt == 2) {
    const float power = -0.5f * rho;
    if (power > 0.0f) return false;
    const float g = expf_ref(power);
    h.G = g;
    h.pf = -g;
    h.gsc = -1.0f;  // no per-splat beta: the settings' beta scales dL/dG (CR/backward.cu:1910-1914)
    if (shape > 0.0f) {
      const float demon = 1.0f + shape * g;
      h.G = (1.0f + shape) * g / demon;
      h.gsc = (1.0f + shape) / (demon * demon);
      h.gs = g * (1.0f - g) / (demon * demon);
    }
    return true;
  }
  const float rho_safe = fmaxf(rho, 1e-8f);
  const float pt = powf_ref(rho_safe, 0.5f * shape);
  const float power = -0.5f * pt;
  if (power > 0.0f) return false;
  h.G = expf_ref(power);
  h.pf = -0.5f * shape * h.G * pt / rho_safe;
  h.gs = -0.25f * h.G * pt * logf_ref(rho_safe);
  return true;
}

// The intersection, Gaussian and alpha of a splat at the pixel
// (backward.cu:1700-1790); true for a hit that passes every test of the
// forward.  pre: the pixel is inside and the splat precedes its last
// contributor.
__device__ __forceinline__ bool bwd_hit(const float4& q0, const float4& q1, const float4& q2, float pxf, float pyf,
                                        float beta, bool pre, BwdHit& h, int kt = 0, float shape = 0.0f) {
  const float Tu[3] = {q0.x, q0.y, q0.z}, Tv[3] = {q0.w, q1.x, q1.y}, Tw[3] = {q1.z, q1.w, q2.x};
#pragma unroll
  for (int r = 0; r < 3; r++) {
    h.k[r] = pxf * Tw[r] - Tu[r];
    h.l[r] = pyf * Tw[r] - Tv[r];
  }
  h.pp[0] = h.k[1] * h.l[2] - h.k[2] * h.l[1];
  h.pp[1] = h.k[2] * h.l[0] - h.k[0] * h.l[2];
  h.pp[2] = h.k[0] * h.l[1] - h.k[1] * h.l[0];
  bool act = pre && h.pp[2] != 0.0f;
  h.s[0] = h.s[1] = 0.0f;
  h.d[0] = h.d[1] = 0.0f;
  h.c_d = 0.0f;
  h.G = 0.0f;
  h.demon = 1.0f;
  h.alpha = 0.0f;
  h.use3d = false;
  if (act) {
    h.s[0] = h.pp[0] / h.pp[2];
    h.s[1] = h.pp[1] / h.pp[2];
    const float rho3d = h.s[0] * h.s[0] + h.s[1] * h.s[1];
    h.d[0] = q2.y - pxf;
    h.d[1] = q2.z - pyf;
    const float rho2d = 2.0f * (h.d[0] * h.d[0] + h.d[1] * h.d[1]);
    const float rho = fminf(rho3d, rho2d);
    h.use3d = rho3d <= rho2d;
    h.c_d = h.use3d ? (h.s[0] * Tw[0] + h.s[1] * Tw[1]) + Tw[2] : Tw[2];
    if (kt == 0) {
      const float power = -0.5f * rho;
      act = h.c_d >= 0.2f && power <= 0.0f;
      if (act) {
        h.G = expf_ref(power);
        if (beta > 0.0f) {
          h.demon = (float)(1.0 + (double)(beta * h.G));
          h.G = (float)((1.0 + (double)beta) * (double)h.G / (double)h.demon);
        }
        h.alpha = fminf(0.99f, q2.w * h.G);
        act = h.alpha >= 1.0f / 255.0f;
      }
    } else {
      act = h.c_d >= 0.2f && bwd_kernel_g(kt, rho, shape, h);
      if (act) {
        h.alpha = fminf(0.99f, q2.w * h.G);
        act = h.alpha >= 1.0f / 255.0f;
      }
    }
  }
  return act;
}

// Per-splat gradient contributions of one pixel's hit (zero without one).
struct BwdGrad {
  float gT[9], gH[9], gM[2], gN[3], gO, gK;
};

__device__ __forceinline__ void bwd_grad_zero(BwdGrad& gr) {
#pragma unroll
  for (int r = 0; r < 9; r++) gr.gT[r] = gr.gH[r] = 0.0f;
  gr.gM[0] = gr.gM[1] = 0.0f;
  gr.gN[0] = gr.gN[1] = gr.gN[2] = 0.0f;
  gr.gO = 0.0f;
  gr.gK = 0.0f;
}

// The blending recursion at a hit (T already divided by 1 - alpha) and the
// gradients it sends to the splat (backward.cu:1799-1913): dot is the hit's
// features (or colour) dotted with dL/dpixel, dxyz the gradient of that dot
// product with respect to the intersection point (zero without a grid),
// contributor the splat's index in the tile's list.
template <bool kHash>
__device__ __forceinline__ void bwd_hit_grad(BwdPixel& px, const BwdHit& h, const float4& q1, const float4& q2,
                                             const float4& q3, const float4& q4, const float4& q5, float beta,
                                             uint32_t contributor, float dot, const float dxyz[3], BwdGrad& gr,
                                             int kt = 0) {
  const float T = px.T, alpha = h.alpha, c_d = h.c_d;
  const float Tw[2] = {q1.z, q1.w};
  if constexpr (kHash) {
    if (h.use3d) {
      gr.gH[0] = dxyz[0] * h.s[0]; gr.gH[1] = dxyz[1] * h.s[0]; gr.gH[2] = dxyz[2] * h.s[0];
      gr.gH[3] = dxyz[0] * h.s[1]; gr.gH[4] = dxyz[1] * h.s[1]; gr.gH[5] = dxyz[2] * h.s[1];
    }
    gr.gH[6] = dxyz[0]; gr.gH[7] = dxyz[1]; gr.gH[8] = dxyz[2];
  }
  // colour term of dL/dalpha (backward.cu:1799-1808 as dot products)
  px.acc_dot = px.last_alpha * px.last_dot + (1.f - px.last_alpha) * px.acc_dot;
  px.last_dot = dot;
  float dL_dalpha = dot - px.acc_dot;
  // RENDER_AXUTILITY terms (backward.cu:1815-1855)
  float dL_dz = 0.0f;
  const float m_d = 100.0f / (100.0f - 0.2f) * (1 - 0.2f / c_d);
  const float dmd_dd = (100.0f * 0.2f) / ((100.0f - 0.2f) * c_d * c_d);
  if ((int)contributor == px.median_contributor - 1) dL_dz += px.dL_dmedian;
  const float dL_dweight = (px.final_D2 + m_d * m_d * px.final_A - 2 * m_d * px.final_D) * px.dL_dreg;
  dL_dalpha += dL_dweight - px.last_dL_dT;
  px.last_dL_dT = dL_dweight * alpha + (1 - alpha) * px.last_dL_dT;
  const float dL_dmd = 2.0f * (T * alpha) * (m_d * px.final_A - px.final_D) * px.dL_dreg;
  dL_dz += dL_dmd * dmd_dd;
  px.accum_depth_rec = px.last_alpha * px.last_depth + (1.f - px.last_alpha) * px.accum_depth_rec;
  px.last_depth = c_d;
  dL_dalpha += (c_d - px.accum_depth_rec) * px.dL_ddepth;
  px.accum_alpha_rec = px.last_alpha * 1.0f + (1.f - px.last_alpha) * px.accum_alpha_rec;
  dL_dalpha += (1 - px.accum_alpha_rec) * px.dL_daccum;
  const float nrm[3] = {q3.x, q3.y, q3.z};
#pragma unroll
  for (int ch = 0; ch < 3; ch++) {
    px.accum_normal_rec[ch] = px.last_alpha * px.last_normal[ch] + (1.f - px.last_alpha) * px.accum_normal_rec[ch];
    px.last_normal[ch] = nrm[ch];
    dL_dalpha += (nrm[ch] - px.accum_normal_rec[ch]) * px.dn2[ch];
    gr.gN[ch] = alpha * T * px.dn2[ch];
  }
  dL_dalpha *= T;
  px.last_alpha = alpha;
  float dL_dG = q2.w * dL_dalpha;
  if (kt == 0) {
    if (beta > 0.0f) {
      const float dG_dg = (float)((1.0 + (double)beta) / (double)(h.demon * h.demon));
      dL_dG *= dG_dg;
    }
  } else {
    gr.gK = dL_dalpha * q2.w * h.gs;  // dL/dshape (CR/backward.cu:1864-1909)
    if (kt == 2) {
      // a flex splat without its own beta falls through to the settings'
      // beta factor with demon = 1 (CR/backward.cu:1875, 1910-1914)
      dL_dG *= h.gsc >= 0.0f ? h.gsc : (beta > 0.0f ? (float)(1.0 + (double)beta) : 1.0f);
    }
  }
  dL_dz += alpha * T * px.dL_ddepth;
  float dL_duv[2] = {0.0f, 0.0f};
  if constexpr (kHash) {
    if (h.use3d) {
      dL_duv[0] = dxyz[0] * q4.x + dxyz[1] * q4.y + dxyz[2] * q4.z;
      dL_duv[1] = dxyz[0] * q4.w + dxyz[1] * q5.x + dxyz[2] * q5.y;
    }
  }
  if (h.use3d) {
    const float dG_factor = kt == 0 ? -h.G : h.pf;
    float dL_ds[2] = {dL_dG * dG_factor * h.s[0] + dL_dz * Tw[0], dL_dG * dG_factor * h.s[1] + dL_dz * Tw[1]};
    dL_ds[0] += dL_duv[0];
    dL_ds[1] += dL_duv[1];
    const float dsx_pz = dL_ds[0] / h.pp[2], dsy_pz = dL_ds[1] / h.pp[2];
    const float dp[3] = {dsx_pz, dsy_pz, -(dsx_pz * h.s[0] + dsy_pz * h.s[1])};
    const float* k = h.k;
    const float* l = h.l;
    const float dk[3] = {l[1] * dp[2] - l[2] * dp[1], l[2] * dp[0] - l[0] * dp[2], l[0] * dp[1] - l[1] * dp[0]};
    const float dl[3] = {dp[1] * k[2] - dp[2] * k[1], dp[2] * k[0] - dp[0] * k[2], dp[0] * k[1] - dp[1] * k[0]};
    const float dz_dTw[3] = {h.s[0], h.s[1], 1.0f};
#pragma unroll
    for (int r = 0; r < 3; r++) {
      gr.gT[r] = -dk[r];
      gr.gT[3 + r] = -dl[r];
      gr.gT[6 + r] = px.pxf * dk[r] + px.pyf * dl[r] + dL_dz * dz_dTw[r];
    }
  } else {
    const float dG_factor_2d = kt == 0 ? -h.G * 2.0f : h.pf * 2.0f;
    gr.gM[0] = dL_dG * (dG_factor_2d * h.d[0]);
    gr.gM[1] = dL_dG * (dG_factor_2d * h.d[1]);
    gr.gT[8] = dL_dz;
  }
  gr.gO = h.G * dL_dalpha;
}

// The wave's per-splat sums (every lane takes part; lanes without a hit add
// zeros) and one atomic per wave, splat and value.  gS is the |grad| sum,
// wcol the colour weight (colour path and the per-splat rows), wt the row's
// blend weight and fdot dL/dweight (render modes 7, 12 and 14).
template <bool kHash, int kRows>
__device__ __forceinline__ void bwd_splat_sums(const RenderBwdParams& p, const BwdPixel& px, uint32_t id, bool act,
                                               const BwdGrad& gr, float gS, float wcol, float wt, float fdot) {
  const size_t HW = (size_t)p.W * p.H;
  const float* dpix = px.dpix;
  const bool lead = (threadIdx.x & 63u) == 0u;
#pragma unroll
  for (int r = 0; r < 9; r++) {
    const float v = wave_sum(gr.gT[r]);
    if (lead && v != 0.0f) atomic_add(p.dtransmat + 9 * (size_t)id + r, v);
  }
  if constexpr (kHash) {
#pragma unroll
    for (int r = 0; r < 9; r++) {
      const float v = wave_sum(gr.gH[r]);
      if (lead && v != 0.0f) atomic_add(p.dhomo + 9 * (size_t)id + r, v);
    }
    const float vs = wave_sum(gS);
    if (lead && vs != 0.0f) atomic_add(p.gradsum + id, vs);
    if constexpr (kRows == 1) {
      for (int ch = 0; ch < p.pgd; ch++) {
        const float v = wave_sum(wcol * dpix[(size_t)ch * HW]);
        if (lead && v != 0.0f) atomic_add(p.dcolors + (size_t)id * p.pgd + ch, v);
      }
    } else if constexpr (kRows == 2) {
      float* dc = p.dcolors + (size_t)id * (uint32_t)p.cstride;
      for (int ch = 0; ch < p.pgd + (p.azero ? 0 : p.nfine); ch++) {
        const float v = wave_sum((ch < p.pgd ? wcol : wcol * wt) * dpix[(size_t)ch * HW]);
        if (lead && v != 0.0f) atomic_add(dc + ch, v);
      }
      const float vw = wave_sum(act ? fdot : 0.0f);
      if (lead && vw != 0.0f) atomic_add(dc + p.wslot, vw);
    }
  } else {
    for (int ch = 0; ch < p.C; ch++) {
      const float v = wave_sum(px.inside ? wcol * dpix[(size_t)ch * HW] : 0.0f);
      if (lead && v != 0.0f) atomic_add(p.dcolors + (size_t)id * p.C + ch, v);
    }
  }
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const float v = wave_sum(gr.gM[r]);
    if (lead && v != 0.0f) atomic_add(p.dmean2D + 3 * (size_t)id + r, v);
  }
#pragma unroll
  for (int r = 0; r < 3; r++) {
    const float v = wave_sum(gr.gN[r]);
    if (lead && v != 0.0f) atomic_add(p.dnormal + 3 * (size_t)id + r, v);
  }
  const float vo = wave_sum(gr.gO);
  if (lead && vo != 0.0f) atomic_add(p.dopacity + id, vo);
  if (p.dshapes != nullptr) {
    const float vk = wave_sum(gr.gK);
    if (lead && vk != 0.0f) atomic_add(p.dshapes + id, vk);
  }
}

// Colour path (no grid): the wave walks the staged splats back to front in
// lockstep, every lane one pixel.
__global__ void __launch_bounds__(kBwdThreads) render_backward_colour_kernel(const RenderBwdParams p) {
  __shared__ float4 srec[4][kBwdThreads];
  __shared__ uint32_t sid[kBwdThreads];
  __shared__ float sshape[kBwdThreads];  // kernel types 1-3: record[26]

  const uint32_t tile = p.tile_order[blockIdx.x];  // the forward's order: heaviest tiles first
  const uint2 range = reinterpret_cast<const uint2*>(p.ranges)[tile];
  const size_t HW = (size_t)p.W * p.H;
  BwdPixel px;
  bwd_pixel_init(p, tile, px);
  const uint32_t total = range.y - range.x;
  for (uint32_t done_n = 0; done_n < total; done_n += kBwdThreads) {
    const uint32_t n = min((uint32_t)kBwdThreads, total - done_n);
    __syncthreads();
    if (threadIdx.x < n) {
      const uint32_t e = range.y - 1u - done_n - threadIdx.x;
      const uint32_t id = p.point_list[e];
      const float4* rec = reinterpret_cast<const float4*>(p.records) + 8 * (size_t)id;
#pragma unroll
      for (int c = 0; c < 4; c++) srec[c][threadIdx.x] = rec[c];
      sid[threadIdx.x] = id;
      sshape[threadIdx.x] = p.kernel_type != 0 ? rec[6].z : 0.0f;
    }
    __syncthreads();
    for (uint32_t j = 0; j < n; j++) {
      const uint32_t contributor = total - 1u - done_n - j;
      const float4 q0 = srec[0][j], q1 = srec[1][j], q2 = srec[2][j], q3 = srec[3][j];
      const uint32_t id = sid[j];
      BwdHit h;
      const bool act = bwd_hit(q0, q1, q2, px.pxf, px.pyf, p.beta, px.inside && contributor < px.last_contributor, h,
                               p.kernel_type, sshape[j]);
      BwdGrad gr;
      bwd_grad_zero(gr);
      float wcol = 0.0f;
      if (act) {
        px.T = px.T / (1.f - h.alpha);
        const float wgt = h.alpha * px.T;
        const float* col = p.colors + (size_t)id * p.C;
        float dot = 0.0f;
        for (int ch = 0; ch < p.C; ch++) dot += col[ch] * px.dpix[(size_t)ch * HW];
        wcol = wgt;
        const float dxyz[3] = {0.0f, 0.0f, 0.0f};
        bwd_hit_grad<false>(px, h, q1, q2, q3, q3, q3, p.beta, contributor, dot, dxyz, gr, p.kernel_type);
      }
      if (__ballot(act) != 0ull) bwd_splat_sums<false, 0>(p, px, id, act, gr, 0.0f, wcol, 0.0f, 0.0f);
    }
  }
}

// Grid path.  A wave walks a batch of staged splats in segments of three
// passes:
//  1. geometry: the splats in lockstep, every lane one pixel; a hit with grid
//     levels queues (grid coordinate, weight, grad_scale, owner lane, level
//     count) in the wave's LDS queue, and every splat with a hit in the wave
//     is listed with its hit and queue masks.  The segment ends when the
//     queue could overflow at the next splat;
//  2. grid: the queued hits spread one per lane, so the table gathers, the
//     feature recomputation, dL/dxyz and the table-gradient scatter run with
//     every lane busy; each hit's (dot, dxyz) replaces its queue entry;
//  3. recursion: the listed splats again, in the same order, with the
//     blending recursion per pixel and the per-splat wave sums.
// kRows 1: render mode 4, per-splat feature rows (p.colors, p.pgd wide) ahead
// of the grid's channels (CR/backward.cu:987-1040).  kRows 2: render mode 12
// training, rows of p.cstride floats ending with the blend weight (p.wslot):
// p.pgd coarse channels from the row, then p.nfine channels blended
// weight * row + (1 - weight) * grid (CR/backward.cu:1425-1520); with p.azero,
// render mode 14 training: rows [pgd | weight], then weight * grid over p.nfine
// channels when the weight is > 1e-6 (CR/backward.cu:1521-1590).
// Grid inputs of a hit (T already divided): the intersection point xyz, the
// level count (0: no lookup) and, in render modes 12 and 14, the row's blend
// weight wt (mode 14 skips the grid at a weight <= 1e-6).
template <int kRows>
__device__ __forceinline__ uint32_t bwd_hit_levels(const RenderBwdParams& p, const BwdHit& h, const float4& q3,
                                                   const float4& q4, const float4& q5, const float4& q6, uint32_t id,
                                                   float xyz[3], float& wt) {
  if (h.use3d) {
    xyz[0] = h.s[0] * q4.x + h.s[1] * q4.w + q5.z;
    xyz[1] = h.s[0] * q4.y + h.s[1] * q5.x + q5.w;
    xyz[2] = h.s[0] * q4.z + h.s[1] * q5.y + q6.x;
  } else {
    xyz[0] = q5.z; xyz[1] = q5.w; xyz[2] = q6.x;
  }
  const uint32_t ap = __float_as_uint(q3.w);
  const uint32_t maxl = ap < p.grid.L ? ap : p.grid.L;
  float u[3], grad_scale;
  uint32_t lane_levels = grid_coord_bwd(p.grid, xyz, u, grad_scale) ? maxl : 0u;
  wt = 0.0f;
  if constexpr (kRows == 2) {
    wt = p.colors[(size_t)id * (uint32_t)p.cstride + p.wslot];
    if (p.azero && !(wt > 1e-6f)) lane_levels = 0u;
  }
  return lane_levels;
}

constexpr int kBwdQueue = 256;  // queued grid hits per wave
constexpr int kBwdList = 128;   // listed splats per wave and segment
constexpr int kBwdWaves = kBwdThreads / 64;

// Three workgroups per CU (51.5 KB of LDS each) where the registers allow:
// F <= 4 fits 168 VGPRs without spills, F = 8 keeps two.
template <int F, int kRows>
__global__ void __launch_bounds__(kBwdThreads) __attribute__((amdgpu_waves_per_eu(F <= 4 ? 3 : 2)))
render_backward_kernel(const RenderBwdParams p) {
  __shared__ float4 srec[kBwdChunks][kBwdThreads];
  __shared__ uint32_t sid[kBwdThreads];
  __shared__ float4 hq[kBwdWaves][kBwdQueue];       // (xyz, w), then (dot, dxyz)
  __shared__ uint16_t hmeta[kBwdWaves][kBwdQueue];  // owner lane | level count << 6
  __shared__ uint64_t lact[kBwdWaves][kBwdList];
  __shared__ uint8_t lj[kBwdWaves][kBwdList];

  const uint32_t tile = p.tile_order[blockIdx.x];  // the forward's order: heaviest tiles first
  const uint2 range = reinterpret_cast<const uint2*>(p.ranges)[tile];
  const size_t HW = (size_t)p.W * p.H;
  const uint32_t lane = threadIdx.x & 63u, wid = threadIdx.x >> 6;
  const uint64_t lt = lane == 0u ? 0ull : (~0ull >> (64u - lane));
  BwdPixel px;
  bwd_pixel_init(p, tile, px);
  const uint32_t tx = tile % p.gx, ty = tile / p.gx;
  const GridParams& g = p.grid;
  const nest_i32x4 rsrc = table_rsrc_rows<F, false>(g.table, g.table_rows);
  const size_t grid_ch = kRows ? (size_t)p.pgd * HW : 0;  // first grid channel of dL/dpixel

  const uint32_t total = range.y - range.x;
  for (uint32_t done_n = 0; done_n < total; done_n += kBwdThreads) {
    const uint32_t n = min((uint32_t)kBwdThreads, total - done_n);
    __syncthreads();
    if (threadIdx.x < n) {
      const uint32_t e = range.y - 1u - done_n - threadIdx.x;
      const uint32_t id = p.point_list[e];
      const float4* rec = reinterpret_cast<const float4*>(p.records) + 8 * (size_t)id;
#pragma unroll
      for (int c = 0; c < kBwdChunks; c++) srec[c][threadIdx.x] = rec[c];
      sid[threadIdx.x] = id;
    }
    __syncthreads();
    for (uint32_t j0 = 0; j0 < n;) {
      // 1. geometry
      float T1 = px.T;
      uint32_t cnt = 0, nl = 0, j = j0;
      while (j < n) {
        const uint32_t contributor = total - 1u - done_n - j;
        const float4 q0 = srec[0][j], q1 = srec[1][j], q2 = srec[2][j];
        BwdHit h;
        const bool act =
            bwd_hit(q0, q1, q2, px.pxf, px.pyf, p.beta, px.inside && contributor < px.last_contributor, h,
                    p.kernel_type, srec[6][j].z);
        float xyz[3] = {0.0f, 0.0f, 0.0f}, hw = 0.0f;
        uint32_t lane_levels = 0u;
        if (act) {
          T1 = T1 / (1.f - h.alpha);
          const float wgt = h.alpha * T1;
          float wt;
          lane_levels = bwd_hit_levels<kRows>(p, h, srec[3][j], srec[4][j], srec[5][j], srec[6][j], sid[j], xyz, wt);
          // the grid's share of the gradient: (1 - weight) of it in mode 12,
          // weight times it in mode 14
          hw = kRows == 2 ? wgt * (p.azero ? wt : 1.0f - wt) : wgt;
        }
        const bool push = lane_levels > 0u;
        const uint64_t m_act = __ballot(act), m_push = __ballot(push);
        if (m_act != 0ull) {
          if (lane == 0u) {
            lact[wid][nl] = m_act;
            lj[wid][nl] = (uint8_t)j;
          }
          nl++;
        }
        if (push) {
          const uint32_t slot = cnt + (uint32_t)__popcll(m_push & lt);
          hq[wid][slot] = make_float4(xyz[0], xyz[1], xyz[2], hw);
          hmeta[wid][slot] = (uint16_t)(lane | (lane_levels << 6));
        }
        cnt += (uint32_t)__popcll(m_push);
        j++;
        if (cnt > (uint32_t)(kBwdQueue - 64) || nl == (uint32_t)kBwdList) break;
      }
      __builtin_amdgcn_wave_barrier();
      // 2. grid: table gradient, features' dot product and dL/dxyz per hit
      for (uint32_t r0 = 0; r0 < cnt; r0 += 64u) {
        const uint32_t e = r0 + lane;
        const bool on = e < cnt;
        float u[3] = {0.0f, 0.0f, 0.0f}, gsc = 0.0f, w = 0.0f;
        uint32_t lev = 0u;
        const float* dp = p.dL_dpix;
        if (on) {
          const float4 q = hq[wid][e];
          const float xyz[3] = {q.x, q.y, q.z};
          w = q.w;
          grid_coord_bwd(g, xyz, u, gsc);  // inside the grid: the hit was queued
          const uint32_t m = hmeta[wid][e];
          lev = m >> 6;
          const uint32_t t = (wid << 6) | (m & 63u);  // the owner's thread
          dp = p.dL_dpix + ((size_t)(ty * kTile + (t >> 4)) * p.W + tx * kTile + (t & 15u)) + grid_ch;
        }
        float dot, dxyz[3];
        // the chunk's queue entries (read above, rewritten below) stage the
        // table-gradient atomics meanwhile
        hash_backward_wave<F>(g, rsrc, u, gsc, lev, w, dp, HW, p.dtable, reinterpret_cast<uint32_t*>(&hq[wid][r0]),
                              dot, dxyz);
        if (on) hq[wid][e] = make_float4(dot, dxyz[0], dxyz[1], dxyz[2]);
      }
      __builtin_amdgcn_wave_barrier();
      // 3. recursion and per-splat sums over the listed splats
      uint32_t qbase = 0;
      for (uint32_t i = 0; i < nl; i++) {
        const uint32_t jj = lj[wid][i];
        const uint64_t m_act = lact[wid][i];
        const bool act = ((m_act >> lane) & 1ull) != 0ull;
        const uint32_t contributor = total - 1u - done_n - jj;
        const float4 q0 = srec[0][jj], q1 = srec[1][jj], q2 = srec[2][jj], q3 = srec[3][jj];
        const float4 q4 = srec[4][jj], q5 = srec[5][jj];
        const uint32_t id = sid[jj];
        BwdHit h;
        bwd_hit(q0, q1, q2, px.pxf, px.pyf, p.beta, act, h, p.kernel_type, srec[6][jj].z);
        bool pushed = false;  // the hit's queue entry, as in the geometry pass
        if (act) {
          float xyz[3], wt0;
          pushed = bwd_hit_levels<kRows>(p, h, q3, q4, q5, srec[6][jj], id, xyz, wt0) > 0u;
        }
        const uint64_t m_push = __ballot(pushed);
        BwdGrad gr;
        bwd_grad_zero(gr);
        float gS = 0.0f, wcol = 0.0f, wt = 0.0f, fdot = 0.0f;
        if (act) {
          px.T = px.T / (1.f - h.alpha);
          const float wgt = h.alpha * px.T;
          gS = wgt * px.sum_abs;
          float rdot = 0.0f, dot = 0.0f, dxyz[3] = {0.0f, 0.0f, 0.0f};
          if (pushed) {
            const float4 r = hq[wid][qbase + (uint32_t)__popcll(m_push & lt)];
            dot = r.x; dxyz[0] = r.y; dxyz[1] = r.z; dxyz[2] = r.w;
          }
          if constexpr (kRows == 1) {
            const float* row = p.colors + (size_t)id * p.pgd;
            for (int ch = 0; ch < p.pgd; ch++) rdot += row[ch] * px.dpix[(size_t)ch * HW];
            wcol = wgt;
            dot += rdot;
          } else if constexpr (kRows == 2) {
            // dot is grid . dpix over the fine channels; the hit's features are
            // the coarse rows and weight * row + (1 - weight) * grid
            const float* row = p.colors + (size_t)id * (uint32_t)p.cstride;
            wt = row[p.wslot];
            for (int ch = 0; ch < p.pgd; ch++) rdot += row[ch] * px.dpix[(size_t)ch * HW];
            if (!p.azero)
              for (int i2 = 0; i2 < p.nfine; i2++) fdot += row[p.pgd + i2] * px.dpix[(size_t)(p.pgd + i2) * HW];
            wcol = wgt;
            const float hdot = dot;
            if (p.azero) {  // mode 14: coarse rows, then weight * grid
              dot = rdot + wt * hdot;
              fdot = wgt * hdot;  // dL/dweight
            } else {
              dot = rdot + wt * fdot + (1.0f - wt) * hdot;
              fdot = wgt * (fdot - hdot);  // dL/dweight
              if (p.wsig) fdot = fdot * wt * (1.0f - wt);  // mode 7: dL/dlogit of weight = sigmoid(logit)
            }
          }
          bwd_hit_grad<true>(px, h, q1, q2, q3, q4, q5, p.beta, contributor, dot, dxyz, gr, p.kernel_type);
        }
        qbase += (uint32_t)__popcll(m_push);
        bwd_splat_sums<true, kRows>(p, px, id, act, gr, gS, wcol, wt, fdot);
      }
      __builtin_amdgcn_wave_barrier();
      j0 = j;
    }
  }
}

template <int F, int kRows = 0>
hipError_t launch_bwd_one(const RenderBwdParams& p, hipStream_t s) {
  hipLaunchKernelGGL((render_backward_kernel<F, kRows>), dim3(p.ntiles), dim3(kBwdThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_bwd_colour(const RenderBwdParams& p, hipStream_t s) {
  hipLaunchKernelGGL(render_backward_colour_kernel, dim3(p.ntiles), dim3(kBwdThreads), 0, s, p);
  return hipGetLastError();
}

// preprocessCUDA backward (backward.cu:2216-2274) with compute_transmat_aabb
// (:2056-2214) and computeColorFromSH backward (:20-140).
__global__ void __launch_bounds__(256) preprocess_backward_kernel(const PreprocessBwdParams p) {
  const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (idx >= p.P || !(p.radii[idx] > 0)) return;
  const float po[3] = {p.means[3 * (size_t)idx], p.means[3 * (size_t)idx + 1], p.means[3 * (size_t)idx + 2]};
  const float* q = p.rots + 4 * (size_t)idx;
  const float sq = 1.0f / sqrtf(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
  const float qw = q[0] * sq, qx = q[1] * sq, qy = q[2] * sq, qz = q[3] * sq;
  float R[3][3];  // R[col][row]
  R[0][0] = 1.f - 2.f * (qy * qy + qz * qz); R[0][1] = 2.f * (qx * qy + qw * qz); R[0][2] = 2.f * (qx * qz - qw * qy);
  R[1][0] = 2.f * (qx * qy - qw * qz); R[1][1] = 1.f - 2.f * (qx * qx + qz * qz); R[1][2] = 2.f * (qy * qz + qw * qx);
  R[2][0] = 2.f * (qx * qz + qw * qy); R[2][1] = 2.f * (qy * qz - qw * qx); R[2][2] = 1.f - 2.f * (qx * qx + qy * qy);
  const float sc[2] = {p.scales[2 * (size_t)idx], p.scales[2 * (size_t)idx + 1]};
  float Lc[3][3];
#pragma unroll
  for (int r = 0; r < 3; r++) {
    Lc[0][r] = R[0][r] * (1.0f * sc[0]);
    Lc[1][r] = R[1][r] * (1.0f * sc[1]);
    Lc[2][r] = R[2][r];
  }
  const float M[3][4] = {{Lc[0][0], Lc[0][1], Lc[0][2], 0.0f}, {Lc[1][0], Lc[1][1], Lc[1][2], 0.0f},
                         {po[0], po[1], po[2], 1.0f}};
  const float N[3][4] = {{(float)p.W / 2.0f, 0.0f, 0.0f, (float)(p.W - 1) / 2.0f},
                         {0.0f, (float)p.H / 2.0f, 0.0f, (float)(p.H - 1) / 2.0f}, {0.0f, 0.0f, 0.0f, 1.0f}};
  float Pm[3][4];
#pragma unroll
  for (int c = 0; c < 3; c++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float a = p.proj[4 * r + 0] * N[c][0];
      a = a + p.proj[4 * r + 1] * N[c][1];
      a = a + p.proj[4 * r + 2] * N[c][2];
      a = a + p.proj[4 * r + 3] * N[c][3];
      Pm[c][r] = a;
    }
  float Tt[3][3];
#pragma unroll
  for (int c = 0; c < 3; c++)
#pragma unroll
    for (int i = 0; i < 3; i++) {
      float a = M[i][0] * Pm[c][0];
      a = a + M[i][1] * Pm[c][1];
      a = a + M[i][2] * Pm[c][2];
      a = a + M[i][3] * Pm[c][3];
      Tt[c][i] = a;
    }
  const float* v = p.view;
  const float nrm[3] = {v[0] * Lc[2][0] + v[4] * Lc[2][1] + v[8] * Lc[2][2],
                        v[1] * Lc[2][0] + v[5] * Lc[2][1] + v[9] * Lc[2][2],
                        v[2] * Lc[2][0] + v[6] * Lc[2][1] + v[10] * Lc[2][2]};
  const float* dTm = p.dtransmat + 9 * (size_t)idx;
  float dT[9];
#pragma unroll
  for (int r = 0; r < 9; r++) dT[r] = dTm[r];
  float* dm2 = p.dmean2D + 3 * (size_t)idx;
  const float m2x = dm2[0], m2y = dm2[1];
  if (m2x != 0 || m2y != 0) {
    const float tv[3] = {9.0f, 9.0f, -1.0f};
    const float T2sq[3] = {Tt[2][0] * Tt[2][0], Tt[2][1] * Tt[2][1], Tt[2][2] * Tt[2][2]};
    const float dd = tv[0] * T2sq[0] + tv[1] * T2sq[1] + tv[2] * T2sq[2];
    const float inv = 1.0f / dd;
    const float f[3] = {tv[0] * inv, tv[1] * inv, tv[2] * inv};
    float dT0[3], dT1[3], dT3[3], df[3];
#pragma unroll
    for (int r = 0; r < 3; r++) {
      dT0[r] = m2x * f[r] * Tt[2][r];
      dT1[r] = m2y * f[r] * Tt[2][r];
      dT3[r] = m2x * f[r] * Tt[0][r] + m2y * f[r] * Tt[1][r];
      df[r] = m2x * Tt[0][r] * Tt[2][r] + m2y * Tt[1][r] * Tt[2][r];
    }
    const float dL_dd = (float)((double)(df[0] * f[0] + df[1] * f[1] + df[2] * f[2]) * (-1.0 / (double)dd));
#pragma unroll
    for (int r = 0; r < 3; r++) {
      dT3[r] += dL_dd * (tv[r] * Tt[2][r] * 2.0f);
      dT[r] += dT0[r];
      dT[3 + r] += dT1[r];
      dT[6 + r] += dT3[r];
    }
  }
  const float* hh = p.dhomo + 9 * (size_t)idx;
  float dM[3][4];
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float a = Pm[0][r] * dT[0 + i];
      a = a + Pm[1][r] * dT[3 + i];
      a = a + Pm[2][r] * dT[6 + i];
      dM[i][r] = a + (r < 3 ? hh[3 * i + r] : 0.0f);
    }
  const float* gn = p.dnormal + 3 * (size_t)idx;
  const float nlen = sqrtf(nrm[0] * nrm[0] + nrm[1] * nrm[1] + nrm[2] * nrm[2]);
  float gu[3] = {0.0f, 0.0f, 0.0f};
  if (nlen > 1e-7f) {
    const float dot = gn[0] * nrm[0] + gn[1] * nrm[1] + gn[2] * nrm[2];
#pragma unroll
    for (int r = 0; r < 3; r++) gu[r] = (gn[r] - dot * nrm[r] / nlen) / nlen;
  }
  float dtn[3] = {v[0] * gu[0] + v[1] * gu[1] + v[2] * gu[2], v[4] * gu[0] + v[5] * gu[1] + v[6] * gu[2],
                  v[8] * gu[0] + v[9] * gu[1] + v[10] * gu[2]};
  const float pv[3] = {v[0] * po[0] + v[4] * po[1] + v[8] * po[2] + v[12],
                       v[1] * po[0] + v[5] * po[1] + v[9] * po[2] + v[13],
                       v[2] * po[0] + v[6] * po[1] + v[10] * po[2] + v[14]};
  const float cosv = -(pv[0] * nrm[0] + pv[1] * nrm[1] + pv[2] * nrm[2]);
  const float mul = cosv > 0 ? 1.0f : -1.0f;
#pragma unroll
  for (int r = 0; r < 3; r++) dtn[r] = mul * dtn[r];
  float dR[3][3];
#pragma unroll
  for (int r = 0; r < 3; r++) {
    dR[0][r] = dM[0][r] * sc[0];
    dR[1][r] = dM[1][r] * sc[1];
    dR[2][r] = dtn[r];
  }
  float* dq = p.drots + 4 * (size_t)idx;
  dq[0] = 2.f * (qx * (dR[1][2] - dR[2][1]) + qy * (dR[2][0] - dR[0][2]) + qz * (dR[0][1] - dR[1][0]));
  dq[1] = 2.f * (-2.f * qx * (dR[1][1] + dR[2][2]) + qy * (dR[0][1] + dR[1][0]) + qz * (dR[0][2] + dR[2][0]) +
                 qw * (dR[1][2] - dR[2][1]));
  dq[2] = 2.f * (qx * (dR[0][1] + dR[1][0]) - 2.f * qy * (dR[0][0] + dR[2][2]) + qz * (dR[1][2] + dR[2][1]) +
                 qw * (dR[2][0] - dR[0][2]));
  dq[3] = 2.f * (qx * (dR[0][2] + dR[2][0]) + qy * (dR[1][2] + dR[2][1]) - 2.f * qz * (dR[0][0] + dR[1][1]) +
                 qw * (dR[0][1] - dR[1][0]));
  p.dscales[2 * (size_t)idx + 0] = dM[0][0] * R[0][0] + dM[0][1] * R[0][1] + dM[0][2] * R[0][2];
  p.dscales[2 * (size_t)idx + 1] = dM[1][0] * R[1][0] + dM[1][1] * R[1][1] + dM[1][2] * R[1][2];
  float dmean[3] = {dM[2][0], dM[2][1], dM[2][2]};

  if (p.shs) {
    // computeColorFromSH backward (backward.cu:20-140)
    const float C0 = 0.28209479177387814f, C1 = 0.4886025119029199f;
    const float C2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f, -1.0925484305920792f,
                         0.5462742152960396f};
    const float C3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f, 0.3731763325901154f,
                         -0.4570457994644658f, 1.445305721320277f, -0.5900435899266435f};
    const float dir[3] = {po[0] - p.campos[0], po[1] - p.campos[1], po[2] - p.campos[2]};
    const float len = sqrtf(dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2]);
    const float x = dir[0] / len, y = dir[1] / len, z = dir[2] / len;
    const int M = p.sh_coeffs, deg = p.sh_degree;
    const float* sh = p.shs + (size_t)idx * M * 3;
    float gc[3];
#pragma unroll
    for (int c = 0; c < 3; c++)
      gc[c] = p.dcolors[3 * (size_t)idx + c] * (p.clamped[3 * (size_t)idx + c] ? 0.0f : 1.0f);
    float* dsh = p.dshs + (size_t)idx * M * 3;
    float ddx[3] = {0, 0, 0}, ddy[3] = {0, 0, 0}, ddz[3] = {0, 0, 0};
    auto SH = [&](int i, int c) { return sh[3 * i + c]; };
    auto put = [&](int i, float w) {
#pragma unroll
      for (int c = 0; c < 3; c++) dsh[3 * i + c] = w * gc[c];
    };
    put(0, C0);
    if (deg > 0) {
      put(1, -C1 * y); put(2, C1 * z); put(3, -C1 * x);
#pragma unroll
      for (int c = 0; c < 3; c++) { ddx[c] = -C1 * SH(3, c); ddy[c] = -C1 * SH(1, c); ddz[c] = C1 * SH(2, c); }
      if (deg > 1) {
        const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
        put(4, C2[0] * xy); put(5, C2[1] * yz); put(6, C2[2] * (2.f * zz - xx - yy));
        put(7, C2[3] * xz); put(8, C2[4] * (xx - yy));
#pragma unroll
        for (int c = 0; c < 3; c++) {
          ddx[c] += C2[0] * y * SH(4, c) + C2[2] * 2.f * -x * SH(6, c) + C2[3] * z * SH(7, c) + C2[4] * 2.f * x * SH(8, c);
          ddy[c] += C2[0] * x * SH(4, c) + C2[1] * z * SH(5, c) + C2[2] * 2.f * -y * SH(6, c) + C2[4] * 2.f * -y * SH(8, c);
          ddz[c] += C2[1] * y * SH(5, c) + C2[2] * 2.f * 2.f * z * SH(6, c) + C2[3] * x * SH(7, c);
        }
        if (deg > 2) {
          put(9, C3[0] * y * (3.f * xx - yy)); put(10, C3[1] * xy * z); put(11, C3[2] * y * (4.f * zz - xx - yy));
          put(12, C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy)); put(13, C3[4] * x * (4.f * zz - xx - yy));
          put(14, C3[5] * z * (xx - yy)); put(15, C3[6] * x * (xx - 3.f * yy));
#pragma unroll
          for (int c = 0; c < 3; c++) {
            ddx[c] += (C3[0] * SH(9, c) * 3.f * 2.f * xy + C3[1] * SH(10, c) * yz + C3[2] * SH(11, c) * -2.f * xy +
                       C3[3] * SH(12, c) * -3.f * 2.f * xz + C3[4] * SH(13, c) * (-3.f * xx + 4.f * zz - yy) +
                       C3[5] * SH(14, c) * 2.f * xz + C3[6] * SH(15, c) * 3.f * (xx - yy));
            ddy[c] += (C3[0] * SH(9, c) * 3.f * (xx - yy) + C3[1] * SH(10, c) * xz +
                       C3[2] * SH(11, c) * (-3.f * yy + 4.f * zz - xx) + C3[3] * SH(12, c) * -3.f * 2.f * yz +
                       C3[4] * SH(13, c) * -2.f * xy + C3[5] * SH(14, c) * -2.f * yz + C3[6] * SH(15, c) * -3.f * 2.f * xy);
            ddz[c] += (C3[1] * SH(10, c) * xy + C3[2] * SH(11, c) * 4.f * 2.f * yz +
                       C3[3] * SH(12, c) * 3.f * (2.f * zz - xx - yy) + C3[4] * SH(13, c) * 4.f * 2.f * xz +
                       C3[5] * SH(14, c) * (xx - yy));
          }
        }
      }
    }
    for (int i = (deg + 1) * (deg + 1); i < M; i++) put(i, 0.0f);
    const float ddir[3] = {ddx[0] * gc[0] + ddx[1] * gc[1] + ddx[2] * gc[2],
                           ddy[0] * gc[0] + ddy[1] * gc[1] + ddy[2] * gc[2],
                           ddz[0] * gc[0] + ddz[1] * gc[1] + ddz[2] * gc[2]};
    const float sum2 = dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2];
    const float invsum32 = 1.0f / sqrtf(sum2 * sum2 * sum2);
    dmean[0] += ((+sum2 - dir[0] * dir[0]) * ddir[0] - dir[1] * dir[0] * ddir[1] - dir[2] * dir[0] * ddir[2]) * invsum32;
    dmean[1] += (-dir[0] * dir[1] * ddir[0] + (sum2 - dir[1] * dir[1]) * ddir[1] - dir[2] * dir[1] * ddir[2]) * invsum32;
    dmean[2] += (-dir[0] * dir[2] * ddir[0] - dir[1] * dir[2] * ddir[1] + (sum2 - dir[2] * dir[2]) * ddir[2]) * invsum32;
  }
  p.dmeans[3 * (size_t)idx + 0] = dmean[0];
  p.dmeans[3 * (size_t)idx + 1] = dmean[1];
  p.dmeans[3 * (size_t)idx + 2] = dmean[2];
  // densification statistic (backward.cu:2268-2271): the render's dL/dT
  const float depth = p.records[32 * (size_t)idx + 8];
  dm2[0] = (float)((double)(dTm[2] * depth) * 0.5 * (double)(float)p.W);
  dm2[1] = (float)((double)(dTm[5] * depth) * 0.5 * (double)(float)p.H);
}

// kernel_grid_backward + kernel_input_backward (gridencoder.cu:245-366) with
// the dy_dx of kernel_grid (:196-242), D = 3, binary32 tables: one lane per
// point, levels in order, table gradients as float atomics, the input
// gradient summed level by level and written once.
template <int F>
__global__ void __launch_bounds__(256) grid_encode_backward_kernel(const GridEncodeBwdParams p) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= p.B) return;
  const float u[3] = {p.inputs[3 * b], p.inputs[3 * b + 1], p.inputs[3 * b + 2]};
  const bool oob = u[0] < 0 || u[0] > 1 || u[1] < 0 || u[1] > 1 || u[2] < 0 || u[2] > 1;
  float gi[3] = {0.0f, 0.0f, 0.0f};
  if (!oob) {
    const nest_i32x4 rsrc = table_rsrc_rows<F, false>(p.table, p.table_rows);
    const float off = p.align_corners ? 0.0f : 0.5f;
    for (int l = 0; l < p.L; l++) {
      const float scale = p.lv.scale[l];
      float pos[3], der[3];
#pragma unroll
      for (int d = 0; d < 3; d++) {
        const float x = u[d] * scale + off;
        pos[d] = x - (float)f2u_sat(x);
        if (p.interp == 1) {
          der[d] = 6.0f * pos[d] * (1.0f - pos[d]);
          pos[d] = pos[d] * pos[d] * (3.0f - 2.0f * pos[d]);
        } else {
          der[d] = 1.0f;
        }
      }
      LevelCorners cn;
      level_corners<F, false>(p.lv, l, off, 0u, u, cn);
      cn.wx[0] = 1 - pos[0]; cn.wx[1] = pos[0];
      cn.wy[0] = 1 - pos[1]; cn.wy[1] = pos[1];
      cn.wz[0] = 1 - pos[2]; cn.wz[1] = pos[2];
      float gr[F];
#pragma unroll
      for (int f = 0; f < F; f++) gr[f] = p.grad[(size_t)b * p.L * F + (size_t)l * F + f];
      float* dl = p.grad_table + (size_t)p.lv.base[l] * F;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float wk = (1.0f * cn.wx[k & 1]) * cn.wy[(k >> 1) & 1] * cn.wz[k >> 2];
#pragma unroll
        for (int f = 0; f < F; f++) atomic_add(dl + (size_t)cn.idx[k] * F + f, wk * gr[f]);
      }
      if (!p.grad_inputs) continue;
      float vals[8][F];
      corners_load<F, false>(rsrc, cn, vals);
#pragma unroll
      for (int gd = 0; gd < 3; gd++) {
        float rg[F];
#pragma unroll
        for (int f = 0; f < F; f++) rg[f] = 0.0f;
#pragma unroll
        for (int idx = 0; idx < 4; idx++) {
          float wgt = scale;
          int kl = 0;
#pragma unroll
          for (int nd = 0; nd < 2; nd++) {
            const int d = (nd >= gd) ? nd + 1 : nd;
            const int bit = (idx >> nd) & 1;
            wgt *= bit ? pos[d] : 1 - pos[d];
            kl |= bit << d;
          }
          const int kr = kl | (1 << gd);
#pragma unroll
          for (int f = 0; f < F; f++) rg[f] += wgt * (vals[kr][f] - vals[kl][f]) * der[gd];
        }
#pragma unroll
        for (int f = 0; f < F; f++) gi[gd] += gr[f] * rg[f];
      }
    }
  }
  if (p.grad_inputs) {
#pragma unroll
    for (int d = 0; d < 3; d++) p.grad_inputs[3 * b + d] = gi[d];
  }
}

}  // namespace

hipError_t launch_grid_encode_backward(const GridEncodeBwdParams& p, hipStream_t s) {
  if (p.B == 0) return hipSuccess;
  const dim3 grid((unsigned)((p.B + 255) / 256));
  switch (p.F) {
    case 1: hipLaunchKernelGGL(grid_encode_backward_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL(grid_encode_backward_kernel<2>, grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL(grid_encode_backward_kernel<4>, grid, dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL(grid_encode_backward_kernel<8>, grid, dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_render_backward(const RenderBwdParams& p, hipStream_t s) {
  if (p.ntiles == 0) return hipSuccess;
  if (p.wslot >= 0) {
    switch (p.grid.F) {
      case 2: return launch_bwd_one<2, 2>(p, s);
      case 4: return launch_bwd_one<4, 2>(p, s);
      case 8: return launch_bwd_one<8, 2>(p, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.pgd > 0) {
    switch (p.grid.F) {
      case 2: return launch_bwd_one<2, 1>(p, s);
      case 4: return launch_bwd_one<4, 1>(p, s);
      case 8: return launch_bwd_one<8, 1>(p, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.level == 0) return launch_bwd_colour(p, s);
  switch (p.grid.F) {
    case 1: return launch_bwd_one<1>(p, s);
    case 2: return launch_bwd_one<2>(p, s);
    case 4: return launch_bwd_one<4>(p, s);
    case 8: return launch_bwd_one<8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_preprocess_backward(const PreprocessBwdParams& p, hipStream_t s) {
  if (p.P == 0) return hipSuccess;
  hipLaunchKernelGGL(preprocess_backward_kernel, dim3((p.P + 255) / 256), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace nest
