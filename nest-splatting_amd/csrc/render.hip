// Per-tile compositing of 2D surfels with a hash-grid lookup at every
// accepted ray/splat hit.
//
// Semantics: renderCUDAsurfelForward<C, render_mode> of
// submodules/diff-surfel-rasterization/cuda_rasterizer/forward.cu:639-2049
// (state :719-785, batch fetch :791-831, intersection loop :834-971, case 0
// :1127-1145, accumulation :1914-1916, appearance colour :1945-1957, output
// :2008-2048), and query_feature (hashgrid.h:53-212); render modes 4
// (hybrid_features, :1218-1282) and 13 (adaptive_cat_fast, :965-1101) in the
// kMix instantiations.
//
// Layout: one 256-thread workgroup per 16x16 tile, one lane per pixel (four
// 64-lane waves of 16x4 pixels).  The tile's sorted splats are staged in LDS
// in batches of 256 packed 128-byte records (structure-of-arrays float4
// chunks, so a wave reads a record with broadcast ds_read_b128).  Workgroups
// launch heaviest tile first (tile_order_kernel), dealt over the XCDs in runs
// of 16.
//
// Work split inside a wave:
//  - compositing runs splat by splat for all 64 pixels: a whole-wave skip when
//    the wave's pixel block is outside the splat's acceptance bbox, a per-lane
//    rcp-based early reject, then the exact test;
//  - an accepted hit updates the depth/normal/distortion state at once and
//    enqueues (grid coordinate, weight, level count) in a per-lane LDS queue;
//  - when any lane's queue is full the wave drains: up to 64 pending hits,
//    oldest first, are spread one per lane whatever pixel they belong to, so
//    the gathers and the interpolation run with all lanes busy; each pixel's
//    lane then accumulates its own hits in front-to-back order.
#include <type_traits>

#include "hashgrid.h"
#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

// Launch shape, measured on the 1M-splat 1600x1064 L=16 F=4 scene (render ms,
// drain one hit per lane per round):
//   batch 256 / queue 4 / 3 waves per SIMD / 8 corner loads in flight  10.2
//   batch 128 (4 workgroups per CU by LDS), 4 waves, 4 loads in flight 13.1
//   batch 128, queue 8, 3 waves                                        10.2
//   2 waves (more VGPRs), two levels' 16 loads in flight               11.5
// Loads in flight per SIMD count for more than occupancy.  Spreading the
// pending hits over all lanes (drain_compact) then took it to 9.7: a round
// drain keeps only ~47 of 64 lanes busy.
constexpr int kRenderThreads = 256;
constexpr int kBatch = 256;    // splats staged in LDS per batch
constexpr int kRecChunks = 8;  // float4 chunks of the record staged per splat
constexpr int kQueue = 4;      // pending hash lookups per pixel
constexpr int kWaveLanes = 64;

__device__ __forceinline__ uint64_t lanemask_lt64() {
  const uint32_t lane = threadIdx.x & (kWaveLanes - 1);
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Level records of the common grid (LevelQuad as four u32), read through the
// scalar cache.
typedef unsigned int nest_u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(4))) nest_u32x4* LevelQuadPtr;

// Corner indices, weights and level offset of level l at u.  Common grid:
// the level's 16-byte record, read with one scalar load at this point (the
// empty asm makes the pointer opaque per level, so the 16 levels' records are
// not all hoisted into registers kept across the whole kernel).  Other grids:
// the level table in the kernel arguments.
__device__ __forceinline__ nest_u32x4 level_record(LevelQuadPtr lqb, int l) {
  LevelQuadPtr ql = lqb;
  asm volatile("" : "+s"(ql));
  return ql[l];
}

template <int F, bool kHalf, bool kStructured>
__device__ __forceinline__ void level_setup(const GridParams& g, nest_u32x4 r, int l, const float u[3],
                                            LevelCorners& cn) {
  if constexpr (kStructured) {
    LevelQuad q;
    q.scale = __uint_as_float(r.x);
    q.a = r.y;
    q.b = r.z;
    q.soff = r.w;
    quad_corners(q, g.pos_offset, u, cn);
  } else {
    level_corners<F, kHalf>(g.lv, l, g.pos_offset, g.interp, u, cn);
  }
}

// level_setup followed by the corner loads of level l.
template <int F, bool kHalf, bool kStructured>
__device__ __forceinline__ void level_fetch(const GridParams& g, nest_u32x4 r, int l, const float u[3],
                                            nest_i32x4 rsrc, LevelCorners& cn, float vals[8][F]) {
  constexpr bool kPair = (kHalf && F == 4) || (!kHalf && F == 2);
  if constexpr (kStructured && kPair) {
    LevelQuad q;
    q.scale = __uint_as_float(r.x);
    q.a = r.y;
    q.b = r.z;
    q.soff = r.w;
    quad_fetch_pairs<F, kHalf>(q, g.pos_offset, u, rsrc, cn, vals);
  } else {
    level_setup<F, kHalf, kStructured>(g, r, l, u, cn);
    corners_load_r<F, kHalf>(rsrc, cn, vals);
  }
}

// One drain round (any F): every lane with a pending hit looks up its oldest
// one (ring-buffer head) and accumulates each level below its level count;
// lanes with an empty queue idle.
template <int F, int NACC, bool kHalf, bool kStructured>
__device__ __forceinline__ void drain_round(const GridParams& g, nest_i32x4 rsrc, float4 (*hq)[kRenderThreads],
                                            uint8_t (*hl)[kRenderThreads], int& qhead, int& qn, float* acc) {
  if (qn > 0) {
    const float4 e = hq[qhead][threadIdx.x];
    const uint32_t maxl = hl[qhead][threadIdx.x];
    const float u[3] = {e.x, e.y, e.z};
    const LevelQuadPtr lqb = (LevelQuadPtr)g.lq;
#pragma unroll
    for (int l = 0; l < NACC / F; l++) {
      if ((uint32_t)l < maxl) {
        LevelCorners cn;
        nest_u32x4 rec = {0u, 0u, 0u, 0u};
        if constexpr (kStructured) rec = level_record(lqb, l);
        float vals[8][F];
        level_fetch<F, kHalf, kStructured>(g, rec, l, u, rsrc, cn, vals);
        float v[F];
        corners_sum_r<F, kHalf>(cn, vals, v);
#pragma unroll
        for (int f = 0; f < F; f++) acc[l * F + f] = fmaf(v[f], e.w, acc[l * F + f]);
      }
    }
    qhead = (qhead + 1) & (kQueue - 1);
    qn--;
  }
}

// Compacted drain (F <= 4): every lane with a pending hit looks up its own
// oldest hit; lanes whose queues are empty take the other lanes' second,
// third, ... entries, depth-major (every second entry before any third), so
// each lane's share is still the oldest `take` entries of its queue.  A lane
// accumulates its own head's values from registers; a lane looking up another
// lane's hit writes each level's F values into that hit's queue slot, and
// the owner adds them after its head, in queue order, acc = fmaf(v, w, acc).
// Levels at or past a hit's level count give 0, and fmaf(0, w, acc) == acc
// (w is finite and the accumulators never hold -0), as in the round drain.
// isrc is this wave's 64-byte table of moved hits: owner lane | slot << 6,
// indexed by the taking lane's rank among the empty lanes.
template <int F, int NACC, bool kHalf, bool kStructured>
__device__ __forceinline__ void drain_compact(const GridParams& g, nest_i32x4 rsrc, float4 (*hq)[kRenderThreads],
                                              uint8_t (*hl)[kRenderThreads], uint8_t* isrc, int& qhead, int& qn,
                                              float* acc) {
  static_assert(F <= 4, "a level's values fit one queue slot");
  const uint32_t lane = threadIdx.x & (kWaveLanes - 1);
  const uint32_t wbase = threadIdx.x - lane;
  const uint64_t lt = lanemask_lt64();
  const bool head = qn > 0;
  const uint64_t idle = ~__ballot(head);
  const uint32_t nidle = (uint32_t)__popcll(idle);
  uint32_t base = 0;
  int take = head ? 1 : 0;
#pragma unroll
  for (int d = 1; d < kQueue; d++) {
    const uint64_t m = __ballot(qn > d);
    const uint32_t k = base + (uint32_t)__popcll(m & lt);
    if (qn > d && k < nidle) {
      isrc[k] = (uint8_t)(lane | ((uint32_t)((qhead + d) & (kQueue - 1)) << 6));
      take = d + 1;
    }
    base += (uint32_t)__popcll(m);
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t rank = (uint32_t)__popcll(idle & lt);
  const bool moved = !head && rank < base;
  const bool work = head || moved;
  float u[3] = {0.0f, 0.0f, 0.0f};
  uint32_t nlev = 0, col = threadIdx.x, wslot = (uint32_t)qhead;
  if (moved) {
    const uint32_t s = isrc[rank];
    col = wbase + (s & 63u);
    wslot = s >> 6;
  }
  if (work) {
    const float4 e = hq[wslot][col];
    u[0] = e.x;
    u[1] = e.y;
    u[2] = e.z;
    nlev = hl[wslot][col];
  }
  float wd[kQueue];
  const float4* own[kQueue];  // this lane's queue slots, oldest first
#pragma unroll
  for (int d = 0; d < kQueue; d++) {
    own[d] = &hq[(qhead + d) & (kQueue - 1)][threadIdx.x];
    wd[d] = d < take ? own[d]->w : 0.0f;
  }
  __builtin_amdgcn_wave_barrier();
  // Software-pipelined over levels: level l+1's gathers are issued as soon as
  // level l is interpolated (its load registers are free then), so they are
  // in flight during level l's hand-off through LDS and the owners' sums.
  constexpr int kLevels = NACC / F;
  const LevelQuadPtr lqb = (LevelQuadPtr)g.lq;
  LevelCorners cn;
  float vals[8][F];
  bool look = work && 0u < nlev;
  nest_u32x4 rec = {0u, 0u, 0u, 0u}, rec_next = {0u, 0u, 0u, 0u};
  if constexpr (kStructured) rec = level_record(lqb, 0);
  if (look) {
    level_fetch<F, kHalf, kStructured>(g, rec, 0, u, rsrc, cn, vals);
  }
  if constexpr (kStructured) rec_next = level_record(lqb, 1);
#pragma unroll
  for (int l = 0; l < kLevels; l++) {
    nest_u32x4 rec_after = {0u, 0u, 0u, 0u};
    if constexpr (kStructured)
      if (l + 2 < kLevels) rec_after = level_record(lqb, l + 2);
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (look) corners_sum_r<F, kHalf>(cn, vals, v);
    bool next = false;
    if (l + 1 < kLevels) {
      next = work && (uint32_t)(l + 1) < nlev;
      if (next) {
        level_fetch<F, kHalf, kStructured>(g, rec_next, l + 1, u, rsrc, cn, vals);
      }
    }
    if (moved) hq[wslot][col] = make_float4(v[0], v[1], v[2], v[3]);
    if (head) {
#pragma unroll
      for (int f = 0; f < F; f++) acc[l * F + f] = fmaf(v[f], wd[0], acc[l * F + f]);
    }
    look = next;
    rec_next = rec_after;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int d = 1; d < kQueue; d++) {
      if (d < take) {
        const float4 r = *own[d];
        const float rv[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int f = 0; f < F; f++) acc[l * F + f] = fmaf(rv[f], wd[d], acc[l * F + f]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  qhead = (qhead + take) & (kQueue - 1);
  qn -= take;
}

// Compacted drain of the per-splat feature modes (F <= 4): drain_compact's
// item table and hand-off, with output level l holding grid level l - hyb
// and each hit's value at a level computed by drain_mixed's rules.  The
// lookup lane loads the row entries of fast and blend hits along with the
// corner gathers, one level ahead.  Hand-offs run only for the output levels
// that can carry a value, [hyb, hyb + max(L, nfast)).
template <int F, int NACC, bool kHalf, bool kStructured, bool kGs>
__device__ __forceinline__ void drain_compact_mix(const RenderParams& p, nest_i32x4 rsrc,
                                                  float4 (*hq)[kRenderThreads], uint32_t (*hm)[kRenderThreads],
                                                  uint8_t* isrc, int& qhead, int& qn, float* acc) {
  static_assert(F <= 4, "a level's values fit one queue slot");
  const GridParams& g = p.grid;
  const uint32_t lane = threadIdx.x & (kWaveLanes - 1);
  const uint32_t wbase = threadIdx.x - lane;
  const uint64_t lt = lanemask_lt64();
  uint32_t base = 0;
  int take = 0;
#pragma unroll
  for (int d = 0; d < kQueue; d++) {
    const uint64_t m = __ballot(qn > d);
    const uint32_t k = base + (uint32_t)__popcll(m & lt);
    if (qn > d && k < (uint32_t)kWaveLanes) {
      isrc[k] = (uint8_t)(lane | ((uint32_t)((qhead + d) & (kQueue - 1)) << 6));
      take = d + 1;
    }
    base += (uint32_t)__popcll(m);
  }
  const uint32_t items = base < (uint32_t)kWaveLanes ? base : (uint32_t)kWaveLanes;
  __builtin_amdgcn_wave_barrier();
  const bool work = lane < items;
  float u[3] = {0.0f, 0.0f, 0.0f};
  uint32_t nhash = 0, nfeat = 0, col = 0, wslot = 0;
  bool fast = false;
  const float* row = p.colors;
  float wt = 0.0f;
  if (work) {
    const uint32_t s = isrc[lane];
    col = wbase + (s & 63u);
    wslot = s >> 6;
    const float4 e = hq[wslot][col];
    u[0] = e.x;
    u[1] = e.y;
    u[2] = e.z;
    const uint32_t meta = hm[wslot][col];
    nhash = meta & 63u;
    fast = (meta & 64u) != 0u;
    row = p.colors + (size_t)(meta >> 7) * (uint32_t)p.cstride;
    wt = p.wslot >= 0 ? row[p.wslot] : p.wfix;
    row += p.pgd;
    nfeat = fast ? p.nfast : (p.blend ? p.nblend : nhash);
  }
  const bool rows = fast || p.blend != 0;
  float wd[kQueue];
#pragma unroll
  for (int d = 0; d < kQueue; d++) wd[d] = d < take ? hq[(qhead + d) & (kQueue - 1)][threadIdx.x].w : 0.0f;
  __builtin_amdgcn_wave_barrier();
  constexpr int kLevels = NACC / F;
  const int hyb = p.hyb;
  const int lend = hyb + (int)(g.L > p.nfast ? g.L : p.nfast);
  const LevelQuadPtr lqb = (LevelQuadPtr)g.lq;
  LevelCorners cn;
  float vals[8][F];
  float rv[F];
#pragma unroll
  for (int f = 0; f < F; f++) rv[f] = 0.0f;
  bool look = false;
  nest_u32x4 rec = {0u, 0u, 0u, 0u}, rec_next = {0u, 0u, 0u, 0u};
  if constexpr (kStructured) rec = level_record(lqb, 0);
  if (hyb == 0) {
    look = work && !fast && 0u < nhash;
    if (look) {
      level_fetch<F, kHalf, kStructured>(g, rec, 0, u, rsrc, cn, vals);
    }
    if (work && rows && 0u < nfeat) {
#pragma unroll
      for (int f = 0; f < F; f++) rv[f] = row[f];
    }
  }
  if constexpr (kStructured) rec_next = level_record(lqb, hyb <= 1 ? 1 - hyb : 0);
#pragma unroll
  for (int l = 0; l < kLevels; l++) {
    const int gl = l - hyb;
    nest_u32x4 rec_after = {0u, 0u, 0u, 0u};
    if constexpr (kStructured)
      if (l + 2 < kLevels) rec_after = level_record(lqb, gl + 2 >= 0 ? gl + 2 : 0);
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (gl >= 0 && work && (uint32_t)gl < nfeat) {
      float h[F];
#pragma unroll
      for (int f = 0; f < F; f++) h[f] = 0.0f;
      if (look) corners_sum_r<F, kHalf>(cn, vals, h);
#pragma unroll
      for (int f = 0; f < F; f++)
        v[f] = fast ? rv[f] : (p.blend ? fmaf(wt, rv[f], (1.0f - wt) * h[f]) : (kGs ? wt * h[f] : h[f]));
    }
    bool next = false;
    if (l + 1 < kLevels && gl + 1 >= 0) {
      const uint32_t gn = (uint32_t)(gl + 1);
      next = work && !fast && gn < nhash;
      if (next) {
        level_fetch<F, kHalf, kStructured>(g, rec_next, (int)gn, u, rsrc, cn, vals);
      }
      if (work && rows && gn < nfeat) {
#pragma unroll
        for (int f = 0; f < F; f++) rv[f] = row[gn * F + f];
      }
    }
    look = next;
    rec_next = rec_after;
    if (gl >= 0 && l < lend) {
      if (work) hq[wslot][col] = make_float4(v[0], v[1], v[2], v[3]);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int d = 0; d < kQueue; d++) {
        if (d < take) {
          const float4 r = hq[(qhead + d) & (kQueue - 1)][threadIdx.x];
          const float rq[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
          for (int f = 0; f < F; f++) acc[l * F + f] = fmaf(rq[f], wd[d], acc[l * F + f]);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  qhead = (qhead + take) & (kQueue - 1);
  qn -= take;
}

// Drain round of the per-splat feature modes (render modes 4 and 13): every
// lane with a pending hit takes its oldest one.  Output level l holds grid
// level l - hyb.  A queued hit's meta word is splat id << 7 | fast << 6 |
// grid levels to look up; its feature at grid level gl is
//   fast (weight > 0.5 in inference)  the row's own features, gl < nfast;
//   blend (training)                  fmaf(wt, row, (1 - wt) * grid), gl < L,
//                                     grid = 0 past the lookup count;
//   otherwise                         the grid, gl < the lookup count;
// and acc = fmaf(feature, w, acc) in queue order, as the other drains.
template <int F, int NACC, bool kHalf, bool kStructured, bool kGs>
__device__ __forceinline__ void drain_mixed(const RenderParams& p, nest_i32x4 rsrc, float4 (*hq)[kRenderThreads],
                                            uint32_t (*hm)[kRenderThreads], int& qhead, int& qn, float* acc) {
  if (qn > 0) {
    const GridParams& g = p.grid;
    const float4 e = hq[qhead][threadIdx.x];
    const uint32_t meta = hm[qhead][threadIdx.x];
    const uint32_t nhash = meta & 63u;
    const bool fast = (meta & 64u) != 0u;
    const float* row = p.colors + (size_t)(meta >> 7) * (uint32_t)p.cstride;
    const float wt = p.wslot >= 0 ? row[p.wslot] : p.wfix;
    const uint32_t nfeat = fast ? p.nfast : (p.blend ? p.nblend : nhash);
    row += p.pgd;
    const float u[3] = {e.x, e.y, e.z};
    const LevelQuadPtr lqb = (LevelQuadPtr)g.lq;
#pragma unroll
    for (int l = 0; l < NACC / F; l++) {
      const int gl = l - p.hyb;
      if (gl < 0) continue;
      if ((uint32_t)gl < nfeat) {
        float h[F];
#pragma unroll
        for (int f = 0; f < F; f++) h[f] = 0.0f;
        if (!fast && (uint32_t)gl < nhash) {
          LevelCorners cn;
          nest_u32x4 rec = {0u, 0u, 0u, 0u};
          if constexpr (kStructured) rec = level_record(lqb, gl);
          float vals[8][F];
          level_fetch<F, kHalf, kStructured>(g, rec, gl, u, rsrc, cn, vals);
          corners_sum_r<F, kHalf>(cn, vals, h);
        }
#pragma unroll
        for (int f = 0; f < F; f++) {
          float v = h[f];
          if (fast)
            v = row[gl * F + f];
          else if (p.blend)
            v = fmaf(wt, row[gl * F + f], (1.0f - wt) * h[f]);
          else if (kGs)
            v = wt * h[f];
          acc[l * F + f] = fmaf(v, e.w, acc[l * F + f]);
        }
      }
    }
    qhead = (qhead + 1) & (kQueue - 1);
    qn--;
  }
}

// Exact ray/surfel test of pixel (pxf, pyf) against a record's chunks 0-2
// and its rho cut (CR/forward.cu:834-900 for the 2DGS kernel_type 0): the
// homogeneous plane intersection, the 3D/2D rho choice, the near test on the
// intersection depth and alpha = min(0.99, opacity * G).  Returns false when
// the pixel rejects the splat.
struct SplatHit {
  float sx, sy, depth, alpha;
  bool use3d;
};

// kernel_type 1-3 (CR/forward.cu:864-900): alpha from the beta kernel
// opacity * (1 - rho)^shape (rho < 1 only), the Gaussian with the splat's own
// beta activation (float arithmetic, as the reference writes it), or the
// general kernel exp(-0.5 * max(rho, 1e-8)^(shape / 2)).  Returns G, or -1
// for a rejected pair.
__device__ __forceinline__ float kernel_g(int kt, float rho, float shape) {
  if (kt == 1) {
    if (rho >= 1.0f) return -1.0f;
    return powf_ref(1.0f - rho, shape);
  }
  if (kt == 2) {
    const float power = -0.5f * rho;
    if (power > 0.0f) return -1.0f;
    float G = expf_ref(power);
    if (shape > 0.0f) G = (1.0f + shape) * G / (1.0f + shape * G);
    return G;
  }
  const float exponent = 0.5f * shape;
  const float pow_term = powf_ref(fmaxf(rho, 1e-8f), exponent);
  const float power = -0.5f * pow_term;
  if (power > 0.0f) return -1.0f;
  return expf_ref(power);
}

__device__ __forceinline__ bool splat_hit(float4 q0, float4 q1, float4 q2, float cut, float pxf, float pyf, float beta,
                                          SplatHit& h, int kt = 0, const float& shape = 0.0f) {
  const float Tu0 = q0.x, Tu1 = q0.y, Tu2 = q0.z, Tv0 = q0.w;
  const float Tv1 = q1.x, Tv2 = q1.y, Tw0 = q1.z, Tw1 = q1.w;
  const float Tw2 = q2.x;
  const float k0 = pxf * Tw0 - Tu0, k1 = pxf * Tw1 - Tu1, k2 = pxf * Tw2 - Tu2;
  const float l0 = pyf * Tw0 - Tv0, l1 = pyf * Tw1 - Tv1, l2 = pyf * Tw2 - Tv2;
  const float p0 = k1 * l2 - k2 * l1, p1 = k2 * l0 - k0 * l2, p2 = k0 * l1 - k1 * l0;
  if (p2 == 0.0f) return false;
  const float dx = q2.y - pxf, dy = q2.z - pyf;
  const float rho2d = 2.0f * (dx * dx + dy * dy);
  // Per-lane early reject: an rcp-based rho3d within 1e-6 of the exact one,
  // scaled down by 1e-5, above the splat's cut and rho2d above it too means
  // alpha < 1/255 in the exact test.  NaNs take the exact path.
  {
    const float rc = __builtin_amdgcn_rcpf(p2);
    const float sxa = p0 * rc, sya = p1 * rc;
    if ((sxa * sxa + sya * sya) * 0.99999f > cut && rho2d > cut) return false;
  }
  const float sx = p0 / p2, sy = p1 / p2;
  const float rho3d = sx * sx + sy * sy;
  const float rho = fminf(rho3d, rho2d);
  const bool use3d = rho3d <= rho2d;
  const float depth = use3d ? (sx * Tw0 + sy * Tw1) + Tw2 : Tw2;
  if (depth < 0.2f) return false;
  float G;
  if (kt == 0) {
    const float power = -0.5f * rho;
    if (power > 0.0f) return false;
    G = expf_ref(power);
    // (1.0 + beta) * G / (1.0 + beta * G) with float beta and G (CR/forward.cu:915-916): the product
    // beta * G is a float product, the rest double
    if (beta > 0.0f) G = (float)((1.0 + (double)beta) * (double)G / (1.0 + (double)(beta * G)));
  } else {
    G = kernel_g(kt, rho, shape);
    if (G < 0.0f) return false;  // a NaN G goes on, as in the reference (alpha = fminf(0.99, NaN))
  }
  const float alpha = fminf(0.99f, q2.w * G);
  if (alpha < 1.0f / 255.0f) return false;
  h.sx = sx;
  h.sy = sy;
  h.depth = depth;
  h.alpha = alpha;
  h.use3d = use3d;
  return true;
}

// World point of an accepted hit: homotrans columns 0, 1, 3 (record chunks
// 4-6) applied to (sx, sy, 1), or the splat centre when rho2d won.
__device__ __forceinline__ void hit_world(float4 q4, float4 q5, float4 q6, const SplatHit& h, float xyz[3]) {
  if (h.use3d) {
    xyz[0] = h.sx * q4.x + h.sy * q4.w + q5.z;
    xyz[1] = h.sx * q4.y + h.sy * q5.x + q5.w;
    xyz[2] = h.sx * q4.z + h.sy * q5.y + q6.x;
  } else {
    xyz[0] = q5.z;
    xyz[1] = q5.w;
    xyz[2] = q6.x;
  }
}

// Normalisation to [0,1]^3 (hashgrid.h:66-98): affine in normal mode (oob
// outside the grid), the unbounded contraction otherwise.
__device__ __forceinline__ void grid_coord(const GridParams& g, const float xyz[3], float u[3], bool& oob) {
  oob = false;
  if (!g.contract) {
#pragma unroll
    for (int d = 0; d < 3; d++) u[d] = (xyz[d] - g.vmin) * g.inv_size;
    oob = (u[0] < 0 || u[0] > 1 || u[1] < 0 || u[1] > 1 || u[2] < 0 || u[2] > 1);
  } else {
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
  }
}

// Levels queried for a hit.  Levels at or past max_level contribute
// fmaf(0, w, acc) == acc (the accumulators never hold -0), so they are not
// queried.
__device__ __forceinline__ uint8_t hit_levels(bool oob, uint32_t ap, uint32_t L) {
  const uint32_t max_level = oob ? 0u : (ap < L ? ap : L);
  return (uint8_t)(max_level < 255u ? max_level : 255u);
}

// State of an accepted hit between the per-lane test and the converged
// feature block of the render modes 4 and 13.
struct PendingHit {
  bool on = false;
  float w = 0.0f, T = 0.0f;
  SplatHit hit{};
};
struct NoPendingHit {};

// Appearance-level colour of a hit (CR/forward.cu:1945-1957): its first two
// channels; the third only ever adds 0 * w.
__device__ __forceinline__ void appearance_colour(uint32_t ap, float w, float& vis0, float& vis1) {
  float apc0, apc1;
  if (ap <= 4u) {
    apc0 = (float)((double)(uint32_t)(ap - 2u) * 0.5);
    apc1 = 1.0f;
  } else {
    apc0 = 1.0f;
    apc1 = (float)(1.0 - (double)(uint32_t)(ap - 4u) * 0.5);
  }
  vis0 += apc0 * w;
  vis1 += apc1 * w;
}

// Hybrid SH modes (CR/forward.cu:1378-1542): query_feature<false, 3, 3> with
// one level at the hit's world point, zero when it is outside the grid, the
// splat's appearance level is 0 or the grid has no level.
__device__ __forceinline__ void hsh_query(const GridParams& g, const float xyz[3], uint32_t ap, float h[3]) {
  h[0] = h[1] = h[2] = 0.0f;
  if (g.L == 0u) return;
  float u[3];
  bool oob;
  grid_coord(g, xyz, u, oob);
  if (oob || ap == 0u) return;
  LevelCorners cn;
  level_corners<3, false>(g.lv, 0, g.pos_offset, g.interp, u, cn);
  const float* t = static_cast<const float*>(g.table) + (size_t)g.lv.base[0] * 3u;
  float vals[8][3];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float* e = t + (size_t)cn.idx[k] * 3u;
    vals[k][0] = e[0];
    vals[k][1] = e[1];
    vals[k][2] = e[2];
  }
  corners_sum<3>(cn, vals, h);
}

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf_ref(-x)); }

// A hit's channels in the hybrid SH modes, accumulated as fmaf(feat, w, acc):
// mode 8 clamp(clamp(raw + 0.5) + sigmoid(h)), mode 10 sigmoid(raw + h)
// (decompose 2: of h alone, 1: of raw alone), mode 9 the 48 coefficients
// with h added to (decompose 2: in place of) the DC terms 0, 16, 32.
template <int kHsh, int NACC>
__device__ __forceinline__ void hsh_accumulate(const RenderParams& p, const float* row, const float h[3], float w,
                                               float* acc) {
  const int dec = p.hsh_dec;
  if constexpr (kHsh == 9) {
#pragma unroll
    for (int c = 0; c < NACC; c++) {
      float v = row[c];
      if (c % 16 == 0 && c < 48) {
        const float hc = h[c / 16];
        v = dec == 2 ? hc : (dec == 1 ? v : v + hc);
      }
      if (c < p.C) acc[c] = fmaf(v, w, acc[c]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 3; c++) {
      float v;
      if constexpr (kHsh == 8) {
        const float gc = fmaxf(0.0f, fminf(1.0f, row[c] + 0.5f));
        const float sc = sigmoid_ref(h[c]);
        v = dec == 2 ? sc : (dec == 1 ? gc : fmaxf(0.0f, fminf(1.0f, gc + sc)));
      } else {
        v = sigmoid_ref(dec == 2 ? h[c] : (dec == 1 ? row[c] : row[c] + h[c]));
      }
      if (c < p.C) acc[c] = fmaf(v, w, acc[c]);
    }
  }
}

// Surface potentials (render modes 1 and 5, CR/forward.cu:1825-1908): the
// grid's levels at the hit, F = 12 (mode 1) or 15 (mode 5) features per
// level of which the first 12 are four 3-vectors dotted with the splat's
// normal n (fused multiply-adds from 0).  Mode 1 writes max(0, -dot + b) with
// b the row's 4 features of the level (the second grid at the splat centre),
// 4 channels per level; mode 5 max(0, -dot), then the row's 3 colours of the
// level (the same grid's features 12-14 at the centre), 7 per level.  Levels
// past min(ap, L), or all of them outside the grid, have zero features.
template <int kHsh, int NACC>
__device__ __forceinline__ void surface_accumulate(const RenderParams& p, const float xyz[3], uint32_t ap,
                                                   const float4& nrm, const float* row, float w, float* acc) {
  constexpr int F = kHsh == 1 ? 12 : 15, kPer = kHsh == 1 ? 4 : 7, kRow = kHsh == 1 ? 4 : 3;
  const GridParams& g = p.grid;
  float u[3];
  bool oob;
  grid_coord(g, xyz, u, oob);
  const uint32_t maxl = oob ? 0u : (ap < g.L ? ap : g.L);
  const float* t = static_cast<const float*>(g.table);
  const float n[3] = {nrm.x, nrm.y, nrm.z};
#pragma unroll
  for (int l = 0; l < NACC / kPer; l++) {
    if ((uint32_t)l >= g.L) continue;  // (continue, not break: the loop stays fully unrolled)
    float fv[12];
#pragma unroll
    for (int f = 0; f < 12; f++) fv[f] = 0.0f;
    if ((uint32_t)l < maxl) {
      LevelCorners cn;
      level_corners<F, false>(g.lv, l, g.pos_offset, g.interp, u, cn);
      // corners_sum's order (w_k = ((1 * wx) * wy) * wz, fmaf per corner from
      // 0), streamed corner by corner to keep the registers down
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float wk = (1.0f * cn.wx[k & 1]) * cn.wy[(k >> 1) & 1] * cn.wz[k >> 2];
        const float* e = t + ((size_t)g.lv.base[l] + cn.idx[k]) * F;
#pragma unroll
        for (int f = 0; f < 12; f++) fv[f] = fmaf(wk, e[f], fv[f]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float dot = 0.0f;
#pragma unroll
      for (int k = 0; k < 3; k++) dot = fmaf(fv[3 * i + k], n[k], dot);
      const float v = kHsh == 1 ? fmaxf(0.0f, -dot + row[l * kRow + i]) : fmaxf(0.0f, -dot);
      if (l * kPer + i < p.C) acc[l * kPer + i] = fmaf(v, w, acc[l * kPer + i]);
    }
    if constexpr (kHsh == 5) {
#pragma unroll
      for (int c = 0; c < 3; c++)
        if (l * kPer + 4 + c < p.C) acc[l * kPer + 4 + c] = fmaf(row[l * kRow + c], w, acc[l * kPer + 4 + c]);
    }
  }
}

// LDS (32 KB of staged records + 17 KB of queue) allows three workgroups per
// CU; amdgpu_waves_per_eu(3) gives the matching 168-VGPR budget, which holds
// 64 accumulators and eight in-flight 16-byte corner loads.
//
// kMix: render modes 4, 12, 13 (1) and 14 (2, grid levels times the weight):
// per-splat features ahead of the grid's; the
// queue then carries a 32-bit meta word per hit (drain_mixed) in place of
// the level count, 53 KB of LDS in all.
// kKT: the splats' kernel comes from p.kernel_type (1-3 possible); without
// it the kernel is the Gaussian, and the kernel-type branch compiles out.
// kHsh: render modes 8, 9, 10 (one 3-channel grid level) and 1, 5 (surface
// potentials) on the colour path's loop (no queue): each hit looks its grid
// levels up in place.
template <int F, int NACC, bool kHash, bool kHalf, bool kStructured = false, int kMix = 0, bool kKT = false,
          int kHsh = 0>
__global__ void __launch_bounds__(kRenderThreads) __attribute__((amdgpu_waves_per_eu(3, 8)))
render_kernel(const RenderParams p) {
  __shared__ float4 srec[kRecChunks][kBatch];
  __shared__ float4 hq[kHash ? kQueue : 1][kRenderThreads];
  __shared__ uint8_t hl[kHash && !kMix ? kQueue : 1][kRenderThreads];
  __shared__ uint32_t hm[kMix ? kQueue : 1][kMix ? kRenderThreads : 1];
  __shared__ uint8_t isrc[kHash ? kRenderThreads : 1];  // compacted-drain item tables, 64 per wave

  const uint32_t tile = p.tile_order[blockIdx.x];
  const uint32_t tx = tile % p.gx, ty = tile / p.gx;
  const uint32_t px = tx * kTile + (threadIdx.x & 15u);
  const uint32_t py = ty * kTile + (threadIdx.x >> 4);
  const bool inside = px < (uint32_t)p.W && py < (uint32_t)p.H;
  const float pxf = (float)px, pyf = (float)py;
  bool done = !inside;
  // pixel block of this wave: 16 columns x 4 rows
  const uint32_t wid = threadIdx.x / kWaveLanes;
  const float wx0 = (float)(tx * kTile), wx1 = wx0 + 15.0f;
  const float wy0 = (float)(ty * kTile + 4u * wid), wy1 = wy0 + 3.0f;

  const uint2 range = reinterpret_cast<const uint2*>(p.ranges)[tile];

  float T = 1.0f;
  uint32_t contributor = 0, last_contributor = 0, render_number = 0;
  float acc[NACC];
#pragma unroll
  for (int c = 0; c < NACC; c++) acc[c] = 0.0f;
  float N0 = 0.f, N1 = 0.f, N2 = 0.f, vis0 = 0.f, vis1 = 0.f;
  float D = 0.f, M1 = 0.f, M2 = 0.f, distortion = 0.f, median_depth = 0.f, median_contributor = -1.0f;
  float pos_x = 0.f, pos_y = 0.f, pos_z = 0.f;
  const float mfac = 100.0f / (100.0f - 0.2f);

  const GridParams& g = p.grid;
  const uint32_t L = g.L;
  nest_i32x4 rsrc{};
  if constexpr (kHash) rsrc = table_rsrc_rows<F, kHalf>(g.table, g.table_rows);
  int qn = 0, qhead = 0;  // per-lane ring buffer of pending lookups
  // kMix: an accepted hit's feature part waits for the converged block after
  // the per-lane test
  [[maybe_unused]] std::conditional_t<(kMix != 0), PendingHit, NoPendingHit> ph;

  // Batches of 256 splats.  The splat index j is uniform across the wave;
  // lanes that are done skip the body, as the reference's per-lane loop
  // stops.  The wave pauses at a splat after which some lane's queue is full
  // and drains, and the last pass (no splats left, or every pixel of the tile
  // done) drains what remains, so the drain has a single call site.
  uint32_t start = range.x;
  for (;;) {
    const bool all_done = __syncthreads_count(done) == kRenderThreads;
    const bool last = start >= range.y || all_done;
    uint32_t n = 0;
    if (!last) {
      const uint32_t e = start + threadIdx.x;
      if (e < range.y) {
        const uint32_t id = p.point_list[e];
        const float4* rec = reinterpret_cast<const float4*>(p.records) + 8 * (size_t)id;
#pragma unroll
        for (int c = 0; c < kRecChunks; c++) srec[c][threadIdx.x] = rec[c];
        srec[6][threadIdx.x].w = __uint_as_float(id);  // the depth's slot: the render recomputes depth per hit
      }
      __syncthreads();
      n = min((uint32_t)kBatch, range.y - start);
    }
    uint32_t j = 0;
    for (;;) {
    while (j < n) {
      if constexpr (kMix) ph.on = false;
      if (!done) {
      contributor++;
      do {
        // Whole-wave skip: the wave's pixel block lies outside the splat's
        // acceptance bbox, so the alpha test rejects every pixel of it.
        const float4 bb = srec[7][j];
        if (bb.y < wx0 || bb.x > wx1 || bb.w < wy0 || bb.z > wy1) break;
        SplatHit hit;
        if (!splat_hit(srec[0][j], srec[1][j], srec[2][j], srec[6][j].y, pxf, pyf, p.beta, hit,
                       kKT ? p.kernel_type : 0, srec[6][j].z))
          break;
        const float test_T = T * (1 - hit.alpha);
        if (test_T < 0.0001f) {
          done = true;
          break;
        }
        const float w = hit.alpha * T;
        render_number++;
        if (p.max_intersections > 0 && render_number >= p.max_intersections) done = true;

        const float4 q3 = srec[3][j];
        const float depth = hit.depth;
        const float Aa = 1 - T;
        const float m = mfac * (1 - 0.2f / depth);
        distortion += (m * m * Aa + M2 - 2 * m * M1) * w;
        D += depth * w;
        M1 += m * w;
        M2 += m * m * w;
        if (T > 0.5f) {
          median_depth = depth;
          median_contributor = (float)contributor;
        }
        N0 += q3.x * w;
        N1 += q3.y * w;
        N2 += q3.z * w;

        if constexpr (kMix) {
          ph.on = true;
          ph.w = w;
          ph.T = test_T;
          ph.hit = hit;
          break;
        }
        if constexpr (kHsh != 0) {
          float xyz[3];
          hit_world(srec[4][j], srec[5][j], srec[6][j], hit, xyz);
          pos_x += w * xyz[0];
          pos_y += w * xyz[1];
          pos_z += w * xyz[2];
          const uint32_t ap = __float_as_uint(q3.w);
          const uint32_t id = __float_as_uint(srec[6][j].w);
          const float* row = p.colors + (size_t)id * (uint32_t)p.cstride;
          if constexpr (kHsh == 1 || kHsh == 5) {
            surface_accumulate<kHsh, NACC>(p, xyz, ap, q3, row, w, acc);
          } else {
            float h[3];
            if (p.hsh_dec != 1)
              hsh_query(g, xyz, ap, h);
            else
              h[0] = h[1] = h[2] = 0.0f;
            hsh_accumulate<kHsh, NACC>(p, row, h, w, acc);
          }
          appearance_colour(ap, w, vis0, vis1);
        } else if constexpr (!kHash) {
          const uint32_t id = __float_as_uint(srec[6][j].w);
          const float* col = p.colors + (size_t)id * p.C;
#pragma unroll
          for (int c = 0; c < NACC; c++)
            if (c < p.C) acc[c] = fmaf(col[c], w, acc[c]);
        } else {
          float xyz[3];
          hit_world(srec[4][j], srec[5][j], srec[6][j], hit, xyz);
          pos_x += w * xyz[0];
          pos_y += w * xyz[1];
          pos_z += w * xyz[2];
          const uint32_t ap = __float_as_uint(q3.w);
          float u[3];
          bool oob;
          grid_coord(g, xyz, u, oob);
          const int slot = (qhead + qn) & (kQueue - 1);
          hq[slot][threadIdx.x] = make_float4(u[0], u[1], u[2], w);
          hl[slot][threadIdx.x] = hit_levels(oob, ap, L);
          qn++;
          float apc0, apc1;
          if (ap <= 4u) {
            apc0 = (float)((double)(uint32_t)(ap - 2u) * 0.5);
            apc1 = 1.0f;
          } else {
            apc0 = 1.0f;
            apc1 = (float)(1.0 - (double)(uint32_t)(ap - 4u) * 0.5);
          }
          vis0 += apc0 * w;
          vis1 += apc1 * w;
        }
        T = test_T;
        last_contributor = contributor;
      } while (false);
      }
      if constexpr (kMix) {
        // Render modes 4 and 13: the splat's feature row is read once per wave
        // with one coalesced load (lane k holds entry k), then broadcast lane by
        // lane; a lane's grid lookups go to its queue.
        if (__ballot(ph.on) != 0ull) {
          const uint32_t id = __builtin_amdgcn_readfirstlane(__float_as_uint(srec[6][j].w));
          const float* row = p.colors + (size_t)id * (uint32_t)p.cstride;
          const uint32_t lane = threadIdx.x & (kWaveLanes - 1);
          float mine = lane < (uint32_t)p.nrow ? row[lane] : 0.0f;
          asm volatile("" : "+v"(mine));  // loaded here, with every lane active
          const float wt = p.wslot >= 0 ? row[p.wslot] : 1.0f;
          // fast hits skip the grid: weight > 0.5 in mode 13 inference, >= 0.9 in
          // mode 12 inference (they take the row), < 0.1 in mode 14 inference and
          // <= 1e-6 in mode 14 training (their grid levels stay zero)
          const bool fast = (wt > p.fthr) != (p.fneg != 0);
          if (ph.on) {
            // per-splat channels at once; a fast hit's grid-level channels too
            // when no earlier hit of the pixel is pending
            const bool enq = !(fast && qn == 0);
            const int ndirect = enq ? p.pgd : p.pgd + (int)p.nfast * F;
#pragma unroll
            for (int c = 0; c < NACC; c++) {
              if (c < ndirect) {
                const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), c));
                acc[c] = fmaf(p.wcoarse ? rv * wt : rv, ph.w, acc[c]);
              }
            }
            const uint32_t ap = __float_as_uint(srec[3][j].w);
            float u[3] = {0.0f, 0.0f, 0.0f};
            uint32_t nh = 0u;
            if (!fast || !p.m13) {  // a mode-13 fast hit has no world point
              float xyz[3];
              hit_world(srec[4][j], srec[5][j], srec[6][j], ph.hit, xyz);
              pos_x += ph.w * xyz[0];
              pos_y += ph.w * xyz[1];
              pos_z += ph.w * xyz[2];
              if (!fast) {
                bool oob;
                grid_coord(g, xyz, u, oob);
                nh = hit_levels(oob, ap, L);
              }
            }
            if (enq) {
              const int slot = (qhead + qn) & (kQueue - 1);
              hq[slot][threadIdx.x] = make_float4(u[0], u[1], u[2], ph.w);
              hm[slot][threadIdx.x] = id << 7 | (fast ? 64u : 0u) | nh;
              qn++;
            }
            if (!p.m13) appearance_colour(ap, ph.w, vis0, vis1);
            T = ph.T;
            // render mode 13 leaves the hit loop before the last-contributor update (CR/forward.cu:1097-1100)
            if (!p.m13) last_contributor = contributor;
          }
        }
      }
      j++;
      if (kHash && __ballot(qn == kQueue)) break;
      if (__ballot(!done) == 0) j = n;
    }
    const bool batch_end = j >= n;
    if constexpr (kHash) {
      // whenever a lane is full; at the end, until every queue is empty
      if (__ballot(qn == kQueue) || (last && __ballot(qn > 0))) {
        if constexpr (kMix && F <= 4)
          drain_compact_mix<F, NACC, kHalf, kStructured, kMix == 2>(p, rsrc, hq, hm, isrc + wid * kWaveLanes, qhead,
                                                                    qn, acc);
        else if constexpr (kMix)
          drain_mixed<F, NACC, kHalf, kStructured, kMix == 2>(p, rsrc, hq, hm, qhead, qn, acc);
        else if constexpr (F <= 4)
          drain_compact<F, NACC, kHalf, kStructured>(g, rsrc, hq, hl, isrc + wid * kWaveLanes, qhead, qn, acc);
        else
          drain_round<F, NACC, kHalf, kStructured>(g, rsrc, hq, hl, qhead, qn, acc);
        if (last) continue;
      }
    }
    if (batch_end) break;
    }
    if (last) break;
    start += kBatch;
  }

  if (!inside) return;
  const size_t HW = (size_t)p.W * p.H;
  const size_t pid = (size_t)p.W * py + px;
  p.final_T[pid] = T;
  p.final_T[pid + HW] = M1;
  p.final_T[pid + 2 * HW] = M2;
  p.n_contrib[pid] = last_contributor;
  p.n_contrib[pid + HW] = f2u_sat(median_contributor);
#pragma unroll
  for (int c = 0; c < NACC; c++) {
    if (c < p.C) {
      int oc = c;
      if constexpr (kMix != 0)
        if (c < p.rot_n) oc = (c + p.rot) % p.rot_n;  // render mode 2: the grid's channels first
      p.out_color[(size_t)oc * HW + pid] = acc[c];
    }
  }
  for (int c = NACC; c < p.C; c++) p.out_color[(size_t)c * HW + pid] = 0.0f;
  float* O = p.out_others;
  O[pid + 0 * HW] = D;
  O[pid + 1 * HW] = 1 - T;
  O[pid + 2 * HW] = N0;
  O[pid + 3 * HW] = N1;
  O[pid + 4 * HW] = N2;
  O[pid + 5 * HW] = median_depth;
  O[pid + 6 * HW] = distortion;
  O[pid + 7 * HW] = (float)render_number;
  O[pid + 8 * HW] = pos_x;
  O[pid + 9 * HW] = pos_y;
  O[pid + 10 * HW] = pos_z;
  O[pid + 11 * HW] = vis0;
  O[pid + 12 * HW] = vis1;
  O[pid + 13 * HW] = 0.0f;  // the third appearance channel only ever adds 0 * w
}

// record_transmittance (CR/forward.cu:1961-1964), for training frames that
// ask for it: for every hit that reaches the blend, the reference adds 1 and
// the pixel's transmittance before the hit to the splat's two counters with
// per-pixel atomics.  Which hits reach the blend, and the transmittance they
// see, depend only on the splats' geometry and opacity (the same test as the
// render kernel's, every render mode but 13, whose hits leave the hit loop
// before the record, :1090), so a second pass over the tile's splats
// recomputes them without any feature work and leaves the render kernel's
// loop untouched.  The wave's lanes visit one splat together: their hits are
// summed across the wave and added with one atomic per counter (the same sums
// in another order; the counts are exact).
__global__ void __launch_bounds__(kRenderThreads) record_transmittance_kernel(const RenderParams p) {
  __shared__ float4 sgeo[5][kBatch];  // record chunks 0-2 (transform, xy, opacity), 7 (acceptance bbox) and 6
                                      // (rho cut in y, kernel shape in z, the splat id bits in w)
  const uint32_t tile = blockIdx.x;
  const uint32_t tx = tile % p.gx, ty = tile / p.gx;
  const uint32_t px = tx * kTile + (threadIdx.x & 15u);
  const uint32_t py = ty * kTile + (threadIdx.x >> 4);
  const bool inside = px < (uint32_t)p.W && py < (uint32_t)p.H;
  const float pxf = (float)px, pyf = (float)py;
  const uint32_t wid = threadIdx.x / kWaveLanes, lane = threadIdx.x & (kWaveLanes - 1);
  const float wx0 = (float)(tx * kTile), wx1 = wx0 + 15.0f;
  const float wy0 = (float)(ty * kTile + 4u * wid), wy1 = wy0 + 3.0f;
  const uint2 range = reinterpret_cast<const uint2*>(p.ranges)[tile];
  bool done = !inside;
  float T = 1.0f;
  uint32_t render_number = 0;
  for (uint32_t start = range.x; start < range.y; start += kBatch) {
    if (__syncthreads_count(done) == kRenderThreads) break;
    const uint32_t e = start + threadIdx.x;
    if (e < range.y) {
      const uint32_t id = p.point_list[e];
      const float4* rec = reinterpret_cast<const float4*>(p.records) + 8 * (size_t)id;
      sgeo[0][threadIdx.x] = rec[0];
      sgeo[1][threadIdx.x] = rec[1];
      sgeo[2][threadIdx.x] = rec[2];
      sgeo[3][threadIdx.x] = rec[7];
      const float4 r6 = rec[6];
      sgeo[4][threadIdx.x] = make_float4(r6.x, r6.y, r6.z, __uint_as_float(id));
    }
    __syncthreads();
    const uint32_t n = min((uint32_t)kBatch, range.y - start);
    for (uint32_t j = 0; j < n; j++) {
      bool hit_blend = false;
      float t_before = 0.0f;
      if (!done) {
        do {
          const float4 bb = sgeo[3][j];
          if (bb.y < wx0 || bb.x > wx1 || bb.w < wy0 || bb.z > wy1) break;
          SplatHit hit;
          if (!splat_hit(sgeo[0][j], sgeo[1][j], sgeo[2][j], sgeo[4][j].y, pxf, pyf, p.beta, hit, p.kernel_type,
                         sgeo[4][j].z))
            break;
          const float test_T = T * (1 - hit.alpha);
          if (test_T < 0.0001f) {
            done = true;
            break;
          }
          render_number++;
          if (p.max_intersections > 0 && render_number >= p.max_intersections) done = true;
          hit_blend = true;
          t_before = T;
          T = test_T;
        } while (false);
      }
      const uint64_t m = __ballot(hit_blend);
      if (m != 0ull) {
        float sum = t_before;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, kWaveLanes);
        if (lane == 0u) {
          const uint32_t id = __float_as_uint(sgeo[4][j].w);
          atomicAdd(p.cover_pixels + id, (float)__popcll(m));
          atomicAdd(p.trans_avg + id, sum);
        }
      }
      if (__ballot(!done) == 0ull) break;
    }
  }
}

// query_feature<false, 16 * 4, 4> of grid g at xyz (levels below min(ap, L),
// the rest 0, all 0 outside the grid), for the dual-grid modes' queries away
// from the hit loop: one lane per point, plain entry loads.  Channel c
// (< nout) goes to out[c * stride], added to it with kAdd.
template <bool kHalf, bool kAdd>
__device__ __forceinline__ void grid_point_features(const GridParams& g, const float xyz[3], uint32_t ap, float* out,
                                                    size_t stride, uint32_t nout) {
  float u[3];
  bool oob;
  grid_coord(g, xyz, u, oob);
  const uint32_t maxl = oob ? 0u : (ap < g.L ? ap : g.L);
  for (uint32_t l = 0; l < g.L; l++) {
    float h[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (l < maxl) {
      LevelCorners cn;
      level_corners<4, kHalf>(g.lv, (int)l, g.pos_offset, g.interp, u, cn);
      float vals[8][4];
#pragma unroll
      for (int k = 0; k < 8; k++) load_entry<4, kHalf>(g.table, (size_t)g.lv.base[l] + cn.idx[k], vals[k]);
      corners_sum<4>(cn, vals, h);
    }
#pragma unroll
    for (int f = 0; f < 4; f++) {
      const uint32_t c = 4u * l + (uint32_t)f;
      if (c < nout) {
        float* o = out + (size_t)c * stride;
        *o = kAdd ? *o + h[f] : h[f];
      }
    }
  }
}

// Render modes 2 and 3 (CR/forward.cu:1164-1175, :1197-1208): the second
// grid at each splat's centre, the homotrans translation column.
__global__ void __launch_bounds__(256) centre_rows_kernel(const GridParams g2, int P, const float* __restrict__ homotrans,
                                                          const float* __restrict__ ap_level, float* __restrict__ rows) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P) return;
  const float* Hm = homotrans + 16 * (size_t)i;
  const float pk[3] = {Hm[3], Hm[7], Hm[11]};
  const uint32_t ap = ap_level ? f2u_sat(floorf(ap_level[i])) : 0xffffffffu;
  grid_point_features<false, false>(g2, pk, ap, rows + (size_t)i * g2.L * 4u, 1, g2.L * 4u);
}

// Render mode 5 (CR/forward.cu:1883-1885, :1904-1906): the grid's features
// 12-14 of each level (15 per level) at each splat's centre, into rows
// [P, L * 3].
__global__ void __launch_bounds__(256) centre_rgb_kernel(const GridParams g, int P, const float* __restrict__ homotrans,
                                                         const float* __restrict__ ap_level, float* __restrict__ rows) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P) return;
  const float* Hm = homotrans + 16 * (size_t)i;
  const float pk[3] = {Hm[3], Hm[7], Hm[11]};
  const uint32_t ap = ap_level ? f2u_sat(floorf(ap_level[i])) : 0xffffffffu;
  float u[3];
  bool oob;
  grid_coord(g, pk, u, oob);
  const uint32_t maxl = oob ? 0u : (ap < g.L ? ap : g.L);
  const float* t = static_cast<const float*>(g.table);
  float* out = rows + (size_t)i * g.L * 3u;
  for (uint32_t l = 0; l < g.L; l++) {
    float h[3] = {0.0f, 0.0f, 0.0f};
    if (l < maxl) {
      LevelCorners cn;
      level_corners<15, false>(g.lv, (int)l, g.pos_offset, g.interp, u, cn);
      float vals[8][3];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float* e = t + ((size_t)g.lv.base[l] + cn.idx[k]) * 15u + 12u;
        vals[k][0] = e[0];
        vals[k][1] = e[1];
        vals[k][2] = e[2];
      }
      corners_sum<3>(cn, vals, h);
    }
    out[3 * l + 0] = h[0];
    out[3 * l + 1] = h[1];
    out[3 * l + 2] = h[2];
  }
}

hipError_t launch_centre_rgb(const GridParams& g, int P, const float* homotrans, const float* ap_level, float* rows,
                             hipStream_t s) {
  if (P <= 0) return hipSuccess;
  hipLaunchKernelGGL(centre_rgb_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, s, g, P, homotrans, ap_level,
                     rows);
  return hipGetLastError();
}

hipError_t launch_centre_rows(const GridParams& g2, int P, const float* homotrans, const float* ap_level, float* rows,
                              hipStream_t s) {
  if (P <= 0) return hipSuccess;
  hipLaunchKernelGGL(centre_rows_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, s, g2, P, homotrans, ap_level,
                     rows);
  return hipGetLastError();
}

// Render mode 3 after the loop (CR/forward.cu:1975-2004), one lane per pixel:
// the grid at the blended position pos (out_others 8-10, not divided by
// alpha), appearance level of the tile's first splat when the pixel has a
// contributor, else 0 (no levels), added to channels [0, L * 4).
template <bool kHalf>
__global__ void __launch_bounds__(256) spatial_add_kernel(const RenderParams p, const float* __restrict__ ap_level) {
  const int64_t HW = (int64_t)p.W * p.H;
  const int64_t pid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pid >= HW) return;
  const uint32_t px = (uint32_t)(pid % p.W), py = (uint32_t)(pid / p.W);
  uint32_t pap = 0u;
  if (ap_level != nullptr && p.n_contrib[pid] > 0u) {
    const uint32_t tile = (py / kTile) * p.gx + px / kTile;
    const uint32_t first = p.point_list[p.ranges[2u * tile]];
    pap = f2u_sat(floorf(ap_level[first]));
  }
  const float pos[3] = {p.out_others[pid + 8 * HW], p.out_others[pid + 9 * HW], p.out_others[pid + 10 * HW]};
  grid_point_features<kHalf, true>(p.grid, pos, pap, p.out_color + pid, (size_t)HW, (uint32_t)p.C);
}

hipError_t launch_spatial_add(const RenderParams& p, const float* ap_level, hipStream_t s) {
  const int64_t HW = (int64_t)p.W * p.H;
  if (HW == 0 || p.grid.L == 0) return hipSuccess;
  const dim3 grid((unsigned)((HW + 255) / 256));
  if (p.grid.half)
    hipLaunchKernelGGL(spatial_add_kernel<true>, grid, dim3(256), 0, s, p, ap_level);
  else
    hipLaunchKernelGGL(spatial_add_kernel<false>, grid, dim3(256), 0, s, p, ap_level);
  return hipGetLastError();
}

template <int F, int NACC, bool kHash, bool kHalf, bool kStructured = false, int kMix = 0, bool kKT = false,
          int kHsh = 0>
static hipError_t launch_one(const RenderParams& p, hipStream_t s) {
  hipLaunchKernelGGL((render_kernel<F, NACC, kHash, kHalf, kStructured, kMix, kKT, kHsh>), dim3(p.ntiles),
                     dim3(kRenderThreads), 0, s, p);
  return hipGetLastError();
}

template <int F, bool kHalf, bool kStructured, bool kKT>
static hipError_t launch_hash_levels(const RenderParams& p, hipStream_t s) {
  const uint32_t L = p.grid.L;
  if constexpr (F * 8 <= NEST_MAX_CHANNELS)
    if (L <= 8) return launch_one<F, F * 8, true, kHalf, kStructured, 0, kKT>(p, s);
  if constexpr (F * 16 <= NEST_MAX_CHANNELS)
    if (L <= 16) return launch_one<F, F * 16, true, kHalf, kStructured, 0, kKT>(p, s);
  if constexpr (F * 32 <= NEST_MAX_CHANNELS)
    if (L <= 32) return launch_one<F, F * 32, true, kHalf, kStructured, 0, kKT>(p, s);
  return hipErrorInvalidValue;
}

// Launch order of the render: tiles by descending pair count, in 256 buckets
// of 8 log2(count + 1), so the heaviest tiles start first and the launch ends
// on light ones; workgroup i runs on XCD i % 8, and each XCD takes runs of 16
// consecutive positions, so the heavy tiles are dealt evenly over the XCDs
// while neighbouring tiles of a bucket tend to share an L2 (on the 1M-splat
// frame runs of 16 raised the L2 hit rate from 35% to 50% and cut the HBM
// traffic from 27.7 to 21.4 GB per launch; the render time moved by less
// than run-to-run noise, and runs of 32 and 64 were slower).  (Giving each XCD
// a band of tile rows with an eighth of the pairs, heaviest first within the
// band, raised the L2 hit rate from 35% to 54% on the 1M-splat frame but
// took the render from 6.16 to 6.83 ms: pair counts balance the XCDs' work
// worse than dealing the heaviest tiles round-robin.)  A tile's pixels do
// not depend on when it runs.  One workgroup.
constexpr int kOrderThreads = 1024;
constexpr int kOrderBins = 256;

__device__ __forceinline__ uint32_t order_bin(uint32_t n) {
  const uint32_t b = (uint32_t)(8.0f * log2f((float)n + 1.0f));
  return (uint32_t)(kOrderBins - 1) - (b < (uint32_t)(kOrderBins - 1) ? b : (uint32_t)(kOrderBins - 1));
}

constexpr int kOrderHeld = 16;  // tiles per thread whose bins stay in registers (16384 tiles)

__global__ void __launch_bounds__(kOrderThreads) tile_order_kernel(const uint2* ranges, uint32_t ntiles,
                                                                  uint32_t* order) {
  static_assert(kOrderBins == 4 * kWaveLanes, "four bins per lane in the scan");
  __shared__ uint32_t cnt[kOrderBins];
  for (int b = threadIdx.x; b < kOrderBins; b += kOrderThreads) cnt[b] = 0u;
  // the thread's first kOrderHeld tiles: all range loads in flight at once,
  // their bins kept for the placement below
  uint32_t bin[kOrderHeld];
#pragma unroll
  for (int k = 0; k < kOrderHeld; k++) {
    const uint32_t t = threadIdx.x + (uint32_t)k * kOrderThreads;
    bin[k] = 0xffffffffu;
    if (t < ntiles) {
      const uint2 r = ranges[t];
      bin[k] = order_bin(r.y - r.x);
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kOrderHeld; k++)
    if (bin[k] != 0xffffffffu) atomicAdd(&cnt[bin[k]], 1u);
  for (uint32_t t = threadIdx.x + kOrderHeld * kOrderThreads; t < ntiles; t += kOrderThreads) {
    const uint2 r = ranges[t];
    atomicAdd(&cnt[order_bin(r.y - r.x)], 1u);
  }
  __syncthreads();
  // exclusive scan of the bins by one wave, four per lane
  if (threadIdx.x < kWaveLanes) {
    const uint32_t l = threadIdx.x;
    const uint32_t c0 = cnt[4 * l], c1 = cnt[4 * l + 1], c2 = cnt[4 * l + 2], c3 = cnt[4 * l + 3];
    const uint32_t s = c0 + c1 + c2 + c3;
    uint32_t inc = s;
#pragma unroll
    for (int d = 1; d < kWaveLanes; d <<= 1) {
      const uint32_t o = __shfl_up(inc, d, kWaveLanes);
      if (l >= (uint32_t)d) inc += o;
    }
    const uint32_t ex = inc - s;
    cnt[4 * l] = ex;
    cnt[4 * l + 1] = ex + c0;
    cnt[4 * l + 2] = ex + c0 + c1;
    cnt[4 * l + 3] = ex + c0 + c1 + c2;
  }
  __syncthreads();
  // Position pos of the descending order goes to workgroup b; within each
  // group of 8 * kRun positions, XCD x (workgroups b with b % 8 == x) takes
  // the run of kRun consecutive positions starting at x * kRun.  Positions
  // within a bucket come from LDS atomics, so their tile order is only as
  // ordered as the atomics are served (a wave's lanes hold consecutive
  // tiles); a run then mostly holds nearby tiles, which share an L2.
  constexpr uint32_t kRun = 16u, kGroup = 8u * kRun;
  const uint32_t full = ntiles / kGroup * kGroup;  // the tail keeps pos == b
  auto place = [&](uint32_t t, uint32_t tb) {
    const uint32_t pos = atomicAdd(&cnt[tb], 1u);
    uint32_t b = pos;
    if (pos < full) {
      const uint32_t g = pos / kGroup, w = pos % kGroup;
      b = (g * kRun + w % kRun) * 8u + w / kRun;
    }
    order[b] = t;
  };
#pragma unroll
  for (int k = 0; k < kOrderHeld; k++)
    if (bin[k] != 0xffffffffu) place(threadIdx.x + (uint32_t)k * kOrderThreads, bin[k]);
  for (uint32_t t = threadIdx.x + kOrderHeld * kOrderThreads; t < ntiles; t += kOrderThreads) {
    const uint2 r = ranges[t];
    place(t, order_bin(r.y - r.x));
  }
}

struct LevelQuads {
  LevelQuad q[NEST_MAX_LEVELS];
};

// Copies the level records from the kernel arguments to device memory, where
// the render reads them with scalar loads.
__global__ void level_quads_kernel(LevelQuads lq, uint32_t L, LevelQuad* dst) {
  if (threadIdx.x != 0) return;
#pragma unroll
  for (int l = 0; l < NEST_MAX_LEVELS; l++)
    if ((uint32_t)l < L) dst[l] = lq.q[l];
}

// Accumulators of the per-splat feature modes: the output levels the mode
// writes (hyb + L, or the row's levels in mode 13), 32 or 64 channels.
template <int F, bool kHalf, bool kStructured, bool kKT>
static hipError_t launch_mix_levels(const RenderParams& p, hipStream_t s) {
  const uint32_t need = (uint32_t)p.pgd + (p.grid.L > p.nfast ? p.grid.L : p.nfast) * (uint32_t)F;
  // mode 14 (grid levels times the weight) has its own drains
  if (p.gscale) {
    if (need <= 32u) return launch_one<F, 32, true, kHalf, kStructured, 2, kKT>(p, s);
    if (need <= 64u) return launch_one<F, 64, true, kHalf, kStructured, 2, kKT>(p, s);
    return hipErrorInvalidValue;
  }
  if (need <= 32u) return launch_one<F, 32, true, kHalf, kStructured, 1, kKT>(p, s);
  if (need <= 64u) return launch_one<F, 64, true, kHalf, kStructured, 1, kKT>(p, s);
  return hipErrorInvalidValue;
}

// kKT (kernel types 1-3) takes the general lookup path only.
template <int F, bool kHalf, bool kKT>
static hipError_t launch_hash(const RenderParams& p, hipStream_t s) {
  if (kKT || !p.grid.structured) {
    if constexpr (F >= 2) {
      if (p.mix) return launch_mix_levels<F, kHalf, false, kKT>(p, s);
    }
    return launch_hash_levels<F, kHalf, false, kKT>(p, s);
  }
  if constexpr (!kKT) {
    const GridParams& g = p.grid;
    LevelQuads lq = {};
    for (uint32_t l = 0; l < g.L; l++) {
      LevelQuad& q = lq.q[l];
      q.scale = g.lv.scale[l];
      const bool dense = l < g.n_dense;
      q.a = dense ? g.lv.res1[l] : g.lv.hsize[l] - 1u;
      q.b = dense ? g.lv.res1[l] * g.lv.res1[l] : 0u;
      q.soff = g.lv.base[l] * (uint32_t)(F * (kHalf ? 2 : 4));
    }
    hipLaunchKernelGGL(level_quads_kernel, dim3(1), dim3(64), 0, s, lq, g.L, g.lq);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if constexpr (F >= 2) {
      if (p.mix) return launch_mix_levels<F, kHalf, true, false>(p, s);
    }
    return launch_hash_levels<F, kHalf, true, false>(p, s);
  }
  return hipErrorInvalidValue;
}

template <bool kKT>
static hipError_t launch_render_kind(const RenderParams& p, hipStream_t s) {
  if (p.hsh == 1) return launch_one<1, 64, false, false, false, 0, kKT, 1>(p, s);
  if (p.hsh == 5) return launch_one<1, 63, false, false, false, 0, kKT, 5>(p, s);
  if (p.hsh == 8) return launch_one<1, 3, false, false, false, 0, kKT, 8>(p, s);
  if (p.hsh == 9) return launch_one<1, 48, false, false, false, 0, kKT, 9>(p, s);
  if (p.hsh == 10) return launch_one<1, 3, false, false, false, 0, kKT, 10>(p, s);
  if (p.level == 0 && !p.mix) {
    if (p.C <= 3) return launch_one<1, 3, false, false, false, 0, kKT>(p, s);
    if (p.C <= 16) return launch_one<1, 16, false, false, false, 0, kKT>(p, s);
    if (p.C <= 32) return launch_one<1, 32, false, false, false, 0, kKT>(p, s);
    if (p.C <= 64) return launch_one<1, 64, false, false, false, 0, kKT>(p, s);
    return launch_one<1, 128, false, false, false, 0, kKT>(p, s);
  }
  const bool half = p.grid.half != 0;
  switch (p.grid.F) {
    case 1: return half ? launch_hash<1, true, kKT>(p, s) : launch_hash<1, false, kKT>(p, s);
    case 2: return half ? launch_hash<2, true, kKT>(p, s) : launch_hash<2, false, kKT>(p, s);
    case 4: return half ? launch_hash<4, true, kKT>(p, s) : launch_hash<4, false, kKT>(p, s);
    case 8: return half ? launch_hash<8, true, kKT>(p, s) : launch_hash<8, false, kKT>(p, s);
    default: return hipErrorInvalidValue;
  }
}

static hipError_t launch_render_kernel(const RenderParams& p, hipStream_t s);

hipError_t launch_render(const RenderParams& p, hipStream_t s) {
  if (p.ntiles == 0) return hipSuccess;
  const hipError_t re = launch_render_kernel(p, s);
  if (re != hipSuccess || p.cover_pixels == nullptr || p.m13) return re;
  hipLaunchKernelGGL(record_transmittance_kernel, dim3(p.ntiles), dim3(kRenderThreads), 0, s, p);
  return hipGetLastError();
}

static hipError_t launch_render_kernel(const RenderParams& p, hipStream_t s) {
  hipLaunchKernelGGL(tile_order_kernel, dim3(1), dim3(kOrderThreads), 0, s, reinterpret_cast<const uint2*>(p.ranges),
                     p.ntiles, p.tile_order);
  const hipError_t oe = hipGetLastError();
  if (oe != hipSuccess) return oe;
  if (p.mix && p.grid.F == 1) return hipErrorInvalidValue;
  return p.kernel_type != 0 ? launch_render_kind<true>(p, s) : launch_render_kind<false>(p, s);
}

}  // namespace nest
