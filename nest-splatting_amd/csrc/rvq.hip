// Residual vector-quantisation decode of splat attributes.
//
// No counterpart in the reference: the workload defines per-attribute
// codebooks [stages, K, dim] (float32) and per-splat uint16 indices
// [P, stages]; the decoded value is the bias plus the stage sum taken in
// stage order, (((cb0[i0] + cb1[i1]) + cb2[i2]) + cb3[i3]), in float32.
// Optional activations are those of scene/gaussian_model.py:26-41: exp for
// scales, normalisation for rotations, sigmoid for opacities, with nest_expf
// so that the decoded splats are reproducible on the host.
//
// Two kernels:
//  - rvq_lds_kernel (one launch per attribute, a stage's codebook of at most
//    64 KiB): a workgroup owns 256 * NS splats, keeps their partial sums in
//    registers, and for each stage copies that stage's codebook into LDS with
//    direct-to-LDS loads and gathers its rows from there.  Random 16-byte rows gathered straight from
//    L2 cost ~146 CU-cycles per 64-lane load instruction on gfx950 (the L2 to
//    L1 path returns whole lines), so the LDS copy (one coalesced stream of
//    the codebook per workgroup and stage) is what lets the decode run at HBM
//    speed on the indices and outputs;
//  - rvq_kernel / rvq_batch_kernel (any shape): one lane per splat, one row
//    load per stage from the L2-resident codebooks.
#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

template <int DIM>
__device__ __forceinline__ void load_row(const float* cb, size_t row, float v[DIM]) {
  if constexpr (DIM == 4) {
    const float4 a = reinterpret_cast<const float4*>(cb)[row];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else if constexpr (DIM == 2) {
    const float2 a = reinterpret_cast<const float2*>(cb)[row];
    v[0] = a.x; v[1] = a.y;
  } else {
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = cb[row * DIM + d];
  }
}

// Bias, optional raw copy, activation and store of splat i's stage sum v
// (kVec: one 8/16-byte store, out aligned to 16 bytes).
template <int DIM, bool kVec>
__device__ __forceinline__ void rvq_finish(const RvqParams& p, int64_t i, float v[DIM], bool bad) {
  if (bad) {
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = __int_as_float(0x7fc00000);
  }
  if (p.has_bias) {
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = p.bias[d] + v[d];
  }
  if (p.raw) {
#pragma unroll
    for (int d = 0; d < DIM; d++) p.raw[i * DIM + d] = v[d];
  }
  if (p.activation == 1) {
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = expf_ref(v[d]);
  } else if (p.activation == 2) {
    float ss = 0.0f;
#pragma unroll
    for (int d = 0; d < DIM; d++) ss = (d == 0) ? v[0] * v[0] : ss + v[d] * v[d];
    const float n = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = v[d] / n;
  } else if (p.activation == 3) {
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = 1.0f / (1.0f + expf_ref(-v[d]));
  }
  if constexpr (kVec && DIM == 4) {
    reinterpret_cast<float4*>(p.out)[i] = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (kVec && DIM == 2) {
    reinterpret_cast<float2*>(p.out)[i] = make_float2(v[0], v[1]);
  } else {
#pragma unroll
    for (int d = 0; d < DIM; d++) p.out[i * DIM + d] = v[d];
  }
}

template <int DIM>
__device__ __forceinline__ void rvq_one(const RvqParams& p, int64_t i) {
  float v[DIM];
  const uint16_t* idx = p.idx + i * p.stages;
  bool bad = false;
  for (int s = 0; s < p.stages; s++) {
    const uint32_t k = idx[s];
    float c[DIM];
    if (k < (uint32_t)p.K) {
      load_row<DIM>(p.cb, (size_t)s * p.K + k, c);
    } else {
      bad = true;
#pragma unroll
      for (int d = 0; d < DIM; d++) c[d] = 0.0f;
    }
#pragma unroll
    for (int d = 0; d < DIM; d++) v[d] = (s == 0) ? c[d] : v[d] + c[d];
  }
  rvq_finish<DIM, false>(p, i, v, bad);
}

template <int DIM>
__global__ void __launch_bounds__(256) rvq_kernel(const RvqParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < p.P) rvq_one<DIM>(p, i);
}

// Several attributes in one launch (blockIdx.y picks the attribute): the
// decode of a splat set is a few MB, so one launch instead of three is most
// of its time.
__global__ void __launch_bounds__(256) rvq_batch_kernel(const RvqBatch b) {
  const RvqParams& p = b.a[blockIdx.y];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.P) return;
  switch (p.dim) {
    case 1: rvq_one<1>(p, i); break;
    case 2: rvq_one<2>(p, i); break;
    case 3: rvq_one<3>(p, i); break;
    case 4: rvq_one<4>(p, i); break;
    default: rvq_one<8>(p, i); break;
  }
}

// LDS-staged decode of one attribute with 4 stages (indices as one 8-byte
// load per splat) and K * DIM a multiple of 4.  Splat n of the workgroup's
// chunk is base + n * 256 + t, so index loads and output stores coalesce.
constexpr int kRvqThreads = 256;

template <int DIM>
__device__ __forceinline__ void lds_row(const float* cb, uint32_t k, float c[DIM]) {
  if constexpr (DIM == 4) {
    const float4 a = reinterpret_cast<const float4*>(cb)[k];
    c[0] = a.x; c[1] = a.y; c[2] = a.z; c[3] = a.w;
  } else if constexpr (DIM == 2) {
    const float2 a = reinterpret_cast<const float2*>(cb)[k];
    c[0] = a.x; c[1] = a.y;
  } else {
#pragma unroll
    for (int d = 0; d < DIM; d++) c[d] = cb[k * DIM + d];
  }
}

// A stage's codebook is at most 4096 16-byte chunks (64 KiB), a multiple of
// 64 chunks; each wave copies its 64-chunk runs with direct-to-LDS loads
// (global_load_lds_dwordx4: lane k's 16 bytes land at the run's LDS address
// + 16 k), all in flight at once, so a stage costs one L2 round trip.
constexpr int kRvqMaxChunks = 4096;
typedef __attribute__((address_space(3))) void lds_void;

template <int DIM, int NS>
__global__ void __launch_bounds__(kRvqThreads) rvq_lds_kernel(const RvqParams p) {
  extern __shared__ float4 lds_cb4[];
  const float* lds_cb = reinterpret_cast<const float*>(lds_cb4);
  const int64_t base = (int64_t)blockIdx.x * (kRvqThreads * NS) + threadIdx.x;
  const uint32_t K = (uint32_t)p.K;
  const uint32_t vec4 = K * DIM / 4;  // 16-byte chunks per stage
  const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  // indices of the chunk's splats (HBM), in flight during the first copy
  uint2 ix[NS];
#pragma unroll
  for (int n = 0; n < NS; n++) {
    const int64_t i = base + (int64_t)n * kRvqThreads;
    ix[n] = i < p.P ? reinterpret_cast<const uint2*>(p.idx)[i] : make_uint2(0u, 0u);
  }
  const float4* cb4 = reinterpret_cast<const float4*>(p.cb);
  float v[NS][DIM];
  bool bad[NS];
#pragma unroll
  for (int n = 0; n < NS; n++) bad[n] = false;
#pragma unroll
  for (int s = 0; s < 4; s++) {
    if (s > 0) __syncthreads();  // every lane is done with the previous stage's rows
    const float4* src = cb4 + (size_t)s * vec4;
    for (uint32_t c0 = 64u * wid; c0 < vec4; c0 += 64u * (kRvqThreads / 64))
      __builtin_amdgcn_global_load_lds(src + c0 + lane, (lds_void*)(lds_cb4 + c0), 16, 0, 0);
    __syncthreads();  // waits for the wave's direct loads, then for every wave
#pragma unroll
    for (int n = 0; n < NS; n++) {
      const uint32_t w = (s < 2) ? ix[n].x : ix[n].y;
      uint32_t k = (s & 1) ? (w >> 16) : (w & 0xffffu);
      if (k >= K) {
        bad[n] = true;
        k = 0u;
      }
      float c[DIM];
      lds_row<DIM>(lds_cb, k, c);
#pragma unroll
      for (int d = 0; d < DIM; d++) v[n][d] = (s == 0) ? c[d] : v[n][d] + c[d];
    }
  }
#pragma unroll
  for (int n = 0; n < NS; n++) {
    const int64_t i = base + (int64_t)n * kRvqThreads;
    if (i < p.P) rvq_finish<DIM, true>(p, i, v[n], bad[n]);
  }
}

// The LDS path applies to 4-stage attributes whose stage codebook is whole
// runs of 64 16-byte chunks and fits 64 KiB (K * dim % 256 == 0), with
// aligned codebooks, indices and outputs.
bool rvq_lds_ok(const RvqParams& p) {
  const size_t stage_bytes = (size_t)p.K * p.dim * sizeof(float);
  return p.stages == 4 && (p.dim == 1 || p.dim == 2 || p.dim == 4) && stage_bytes <= (size_t)kRvqMaxChunks * 16 &&
         ((size_t)p.K * p.dim) % 256 == 0 && (reinterpret_cast<uintptr_t>(p.cb) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(p.idx) & 7u) == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0;
}

// Splats per lane: the most that keeps at least 512 workgroups (two per CU),
// capped per dimension so the partial sums fit the registers.
template <int DIM>
static hipError_t launch_rvq_lds_dim(const RvqParams& p, hipStream_t s) {
  const size_t lds = (size_t)p.K * DIM * sizeof(float);
  constexpr int kMax = DIM == 4 ? 8 : 16;
  int ns = kMax;
  while (ns > 2 && (p.P + (int64_t)kRvqThreads * ns - 1) / ((int64_t)kRvqThreads * ns) < 512) ns /= 2;
  const int64_t chunk = (int64_t)kRvqThreads * ns;
  const dim3 grid((unsigned)((p.P + chunk - 1) / chunk));
  switch (ns) {
    case 16:
      if constexpr (kMax >= 16) {
        hipLaunchKernelGGL((rvq_lds_kernel<DIM, 16>), grid, dim3(kRvqThreads), lds, s, p);
        break;
      }
      [[fallthrough]];
    case 8: hipLaunchKernelGGL((rvq_lds_kernel<DIM, 8>), grid, dim3(kRvqThreads), lds, s, p); break;
    case 4: hipLaunchKernelGGL((rvq_lds_kernel<DIM, 4>), grid, dim3(kRvqThreads), lds, s, p); break;
    default: hipLaunchKernelGGL((rvq_lds_kernel<DIM, 2>), grid, dim3(kRvqThreads), lds, s, p); break;
  }
  return hipGetLastError();
}

static hipError_t launch_rvq_lds(const RvqParams& p, hipStream_t s) {
  if (p.P <= 0) return hipSuccess;
  switch (p.dim) {
    case 1: return launch_rvq_lds_dim<1>(p, s);
    case 2: return launch_rvq_lds_dim<2>(p, s);
    default: return launch_rvq_lds_dim<4>(p, s);
  }
}

hipError_t launch_rvq(const RvqParams& p, hipStream_t s) {
  if (p.P <= 0) return hipSuccess;
  if (rvq_lds_ok(p)) return launch_rvq_lds(p, s);
  const dim3 grid((unsigned)((p.P + 255) / 256));
  switch (p.dim) {
    case 1: hipLaunchKernelGGL(rvq_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL(rvq_kernel<2>, grid, dim3(256), 0, s, p); break;
    case 3: hipLaunchKernelGGL(rvq_kernel<3>, grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL(rvq_kernel<4>, grid, dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL(rvq_kernel<8>, grid, dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Fused, persistent decode of several attributes (all 4-stage, on the LDS
// path's shapes): one 1024-thread workgroup per CU (16 waves sharing 128 KiB of LDS), the
// workgroups split between the attributes in proportion to their HBM bytes
// (8-byte index row plus the output row per splat).  An attribute whose four
// stage codebooks fit 128 KiB (dim 1 and 2 at 4096 entries) copies them into
// LDS once per workgroup and keeps them there for all its chunks.  One whose
// stage pairs fit (dim 4: 2 x 64 KiB) holds one pair at a time and
// alternates the pair order from chunk to chunk, so each chunk copies one
// pair, not four stages: an even-numbered chunk gathers stages 0-1 then 2-3,
// an odd one 2-3 (rows kept) then 0-1.  Either way the value is
// ((c0 + c1) + c2) + c3 in that order, as the per-splat kernels sum it.  The
// next chunk's indices are loaded while the current chunk is decoded.
constexpr int kRvqFusedThreads = 1024;
// Splats per lane and chunk: 8 for an attribute that copies stage pairs per
// chunk (the copy is paid once per 8192 splats), 4 for one whose codebooks
// stay resident, whose chunks cost only their HBM bytes, so the workgroup
// split balances at a finer grain (4M splats: 51.2 -> 49.8 us; 2 per lane:
// 54.0 us).
constexpr int kRvqFusedNS = 8;
constexpr int kRvqFusedNSResident = 4;
template <int DIM>
constexpr int rvq_fused_ns() { return DIM == 4 ? kRvqFusedNS : kRvqFusedNSResident; }
constexpr int kRvqFusedChunks = 8192;          // 16-byte LDS chunks per workgroup (128 KiB)

struct RvqFused {
  RvqParams a[kRvqBatchMax];
  int n;
  int wg_first[kRvqBatchMax + 1];  // workgroups [wg_first[k], wg_first[k + 1]) decode attribute k
};

// Copies `chunks` 16-byte chunks (a multiple of 64) from src to the LDS
// array with direct-to-LDS loads, 64 per wave instruction, all in flight.
__device__ __forceinline__ void rvq_copy_lds(const float4* src, uint32_t chunks, float4* lds) {
  const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (uint32_t c0 = 64u * wid; c0 < chunks; c0 += 64u * (kRvqFusedThreads / 64))
    __builtin_amdgcn_global_load_lds(src + c0 + lane, (lds_void*)(lds + c0), 16, 0, 0);
}

// Stage s's codebook index in a splat's index row (four u16 in a uint2);
// an index of K or more reads row 0 and marks the splat bad.
__device__ __forceinline__ uint32_t rvq_stage_index(uint2 w, int s, uint32_t K, bool& bad) {
  const uint32_t x = (s < 2) ? w.x : w.y;
  const uint32_t k = (s & 1) ? (x >> 16) : (x & 0xffffu);
  if (k >= K) {
    bad = true;
    return 0u;
  }
  return k;
}

// Index rows of chunk c (zeros past the end).
template <int NS>
__device__ __forceinline__ void rvq_load_ix(const uint2* idx2, int64_t P, int64_t c, int64_t nchunks, uint2 (&ix)[NS]) {
  const int64_t chunk = (int64_t)kRvqFusedThreads * NS;
#pragma unroll
  for (int n = 0; n < NS; n++) {
    const int64_t i = c * chunk + (int64_t)n * kRvqFusedThreads + threadIdx.x;
    ix[n] = (c < nchunks && i < P) ? idx2[i] : make_uint2(0u, 0u);
  }
}

template <int DIM>
__device__ void rvq_fused_attr(const RvqParams& p, int wg, int nwg, float4* lds4) {
  constexpr int NS = rvq_fused_ns<DIM>();
  const float* lds = reinterpret_cast<const float*>(lds4);
  const uint32_t K = (uint32_t)p.K;
  const uint32_t vec4 = K * DIM / 4;  // 16-byte chunks per stage
  const float* st1 = lds + (size_t)vec4 * 4;  // second stage of a pair
  const bool resident = 4u * vec4 <= (uint32_t)kRvqFusedChunks;
  const int64_t chunk = (int64_t)kRvqFusedThreads * NS;
  const int64_t nchunks = (p.P + chunk - 1) / chunk;
  const float4* cb4 = reinterpret_cast<const float4*>(p.cb);
  const uint2* idx2 = reinterpret_cast<const uint2*>(p.idx);
  uint2 ixn[NS];
  rvq_load_ix<NS>(idx2, p.P, wg, nchunks, ixn);
  if (resident) {
    rvq_copy_lds(cb4, 4u * vec4, lds4);
    __syncthreads();
  }
  int held = -1;  // stage pair in LDS (pair mode): 0 = stages 0-1, 1 = stages 2-3
  for (int64_t c = wg; c < nchunks; c += nwg) {
    uint2 ix[NS];
#pragma unroll
    for (int n = 0; n < NS; n++) ix[n] = ixn[n];
    rvq_load_ix<NS>(idx2, p.P, c + nwg, nchunks, ixn);
    bool bad[NS];
    float v[NS][DIM];
#pragma unroll
    for (int n = 0; n < NS; n++) bad[n] = false;
    if (resident) {
#pragma unroll
      for (int n = 0; n < NS; n++) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
          float r[DIM];
          lds_row<DIM>(lds + (size_t)st * vec4 * 4, rvq_stage_index(ix[n], st, K, bad[n]), r);
#pragma unroll
          for (int d = 0; d < DIM; d++) v[n][d] = (st == 0) ? r[d] : v[n][d] + r[d];
        }
      }
    } else if (held == 1) {
      // stages 2-3 first, their rows kept; then stages 0-1 and the ordered sum
      float r2[NS][DIM], r3[NS][DIM];
#pragma unroll
      for (int n = 0; n < NS; n++) {
        lds_row<DIM>(lds, rvq_stage_index(ix[n], 2, K, bad[n]), r2[n]);
        lds_row<DIM>(st1, rvq_stage_index(ix[n], 3, K, bad[n]), r3[n]);
      }
      __syncthreads();
      rvq_copy_lds(cb4, 2u * vec4, lds4);
      __syncthreads();
      held = 0;
#pragma unroll
      for (int n = 0; n < NS; n++) {
        float r0[DIM], r1[DIM];
        lds_row<DIM>(lds, rvq_stage_index(ix[n], 0, K, bad[n]), r0);
        lds_row<DIM>(st1, rvq_stage_index(ix[n], 1, K, bad[n]), r1);
#pragma unroll
        for (int d = 0; d < DIM; d++) v[n][d] = ((r0[d] + r1[d]) + r2[n][d]) + r3[n][d];
      }
    } else {
      // stages 0-1 (copied unless held), then 2-3
      if (held != 0) {
        __syncthreads();
        rvq_copy_lds(cb4, 2u * vec4, lds4);
        __syncthreads();
      }
#pragma unroll
      for (int n = 0; n < NS; n++) {
        float r0[DIM], r1[DIM];
        lds_row<DIM>(lds, rvq_stage_index(ix[n], 0, K, bad[n]), r0);
        lds_row<DIM>(st1, rvq_stage_index(ix[n], 1, K, bad[n]), r1);
#pragma unroll
        for (int d = 0; d < DIM; d++) v[n][d] = r0[d] + r1[d];
      }
      __syncthreads();
      rvq_copy_lds(cb4 + 2u * vec4, 2u * vec4, lds4);
      __syncthreads();
      held = 1;
#pragma unroll
      for (int n = 0; n < NS; n++) {
        float r2[DIM], r3[DIM];
        lds_row<DIM>(lds, rvq_stage_index(ix[n], 2, K, bad[n]), r2);
        lds_row<DIM>(st1, rvq_stage_index(ix[n], 3, K, bad[n]), r3);
#pragma unroll
        for (int d = 0; d < DIM; d++) v[n][d] = (v[n][d] + r2[d]) + r3[d];
      }
    }
#pragma unroll
    for (int n = 0; n < NS; n++) {
      const int64_t i = c * chunk + (int64_t)n * kRvqFusedThreads + threadIdx.x;
      if (i < p.P) rvq_finish<DIM, true>(p, i, v[n], bad[n]);
    }
  }
}

__global__ void __launch_bounds__(kRvqFusedThreads, 1) rvq_fused_kernel(const RvqFused f) {
  __shared__ float4 lds[kRvqFusedChunks];
  int a = 0;
  while (a + 1 < f.n && (int)blockIdx.x >= f.wg_first[a + 1]) a++;
  const RvqParams& p = f.a[a];
  const int wg = (int)blockIdx.x - f.wg_first[a], nwg = f.wg_first[a + 1] - f.wg_first[a];
  switch (p.dim) {
    case 1: rvq_fused_attr<1>(p, wg, nwg, lds); break;
    case 2: rvq_fused_attr<2>(p, wg, nwg, lds); break;
    default: rvq_fused_attr<4>(p, wg, nwg, lds); break;
  }
}

// The fused path takes attributes on the LDS path's shapes whose stage pair
// fits 128 KiB.
static bool rvq_fused_ok(const RvqParams& p) {
  return rvq_lds_ok(p) && 2ull * (size_t)p.K * p.dim * sizeof(float) <= (size_t)kRvqFusedChunks * 16;
}

static int rvq_device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

hipError_t launch_rvq_batch(const RvqBatch& b, hipStream_t s) {
  // every attribute on the fused path: one persistent launch, one workgroup
  // per CU.  Workgroups are dealt one at a time to the attribute whose
  // finishing time ceil(chunks / workgroups) x (HBM bytes of a chunk) is
  // the largest, so the slowest attribute sets the launch's length with no
  // workgroup left over (at least one per non-empty attribute, none beyond
  // its chunk count).  Counting the rotation codebook's stage-pair copies
  // as well (from L2, 128 KiB per chunk) made 4M splats slower, 0.068 ms
  // against 0.053 ms.
  bool all_fused = b.n > 0;
  for (int k = 0; k < b.n; k++) all_fused = all_fused && rvq_fused_ok(b.a[k]);
  if (all_fused) {
    RvqFused f{};
    f.n = b.n;
    for (int k = 0; k < b.n; k++) f.a[k] = b.a[k];
    const int cus = rvq_device_cus();
    int64_t chunks[kRvqBatchMax], g[kRvqBatchMax];
    double cost[kRvqBatchMax];
    int used = 0;
    for (int k = 0; k < b.n; k++) {
      const RvqParams& p = b.a[k];
      const int64_t cs = (int64_t)kRvqFusedThreads * (p.dim == 4 ? kRvqFusedNS : kRvqFusedNSResident);
      chunks[k] = (p.P + cs - 1) / cs;
      cost[k] = (double)cs * (8 + 4 * p.dim);  // index row + output row per splat
      g[k] = chunks[k] > 0 ? 1 : 0;
      used += (int)g[k];
    }
    while (used < cus) {
      int worst = -1;
      double wt = 0.0;
      for (int k = 0; k < b.n; k++) {
        if (g[k] == 0 || g[k] >= chunks[k]) continue;
        const double t = (double)((chunks[k] + g[k] - 1) / g[k]) * cost[k];
        if (t > wt) { wt = t; worst = k; }
      }
      if (worst < 0) break;
      g[worst]++;
      used++;
    }
    int next = 0;
    for (int k = 0; k < b.n; k++) {
      f.wg_first[k] = next;
      next += (int)g[k];
    }
    f.wg_first[b.n] = next;
    if (next == 0) return hipSuccess;
    hipLaunchKernelGGL(rvq_fused_kernel, dim3((unsigned)next), dim3(kRvqFusedThreads), 0, s, f);
    return hipGetLastError();
  }
  // every attribute on the LDS path: one launch each (their LDS sizes differ)
  bool all_lds = b.n > 0;
  for (int k = 0; k < b.n; k++) all_lds = all_lds && rvq_lds_ok(b.a[k]);
  if (all_lds) {  // one launch per attribute, each with its own codebook's LDS size
    for (int k = 0; k < b.n; k++) {
      const hipError_t e = launch_rvq_lds(b.a[k], s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  int64_t pmax = 0;
  for (int k = 0; k < b.n; k++) pmax = b.a[k].P > pmax ? b.a[k].P : pmax;
  if (pmax <= 0 || b.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(rvq_batch_kernel, dim3((unsigned)((pmax + 255) / 256), (unsigned)b.n), dim3(256), 0, s, b);
  return hipGetLastError();
}

}  // namespace nest
