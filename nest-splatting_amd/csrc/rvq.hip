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
// One lane per splat: the stage indices come in as one 8-byte load, every
// codebook row as one dim*4-byte load (the 448 KiB of codebooks stay in L2).
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
#pragma unroll
  for (int d = 0; d < DIM; d++) p.out[i * DIM + d] = v[d];
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

hipError_t launch_rvq(const RvqParams& p, hipStream_t s) {
  if (p.P <= 0) return hipSuccess;
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

hipError_t launch_rvq_batch(const RvqBatch& b, hipStream_t s) {
  int64_t pmax = 0;
  for (int k = 0; k < b.n; k++) pmax = b.a[k].P > pmax ? b.a[k].P : pmax;
  if (pmax <= 0 || b.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(rvq_batch_kernel, dim3((unsigned)((pmax + 255) / 256), (unsigned)b.n), dim3(256), 0, s, b);
  return hipGetLastError();
}

}  // namespace nest
