// Tile binning: inclusive scan of tiles touched, duplicate-with-keys, a stable
// LSD radix sort of (tile << 32 | depth bits, splat id) pairs and per-tile
// range identification.
//
// Semantics: CR/rasterizer_impl.cu:355 (cub::DeviceScan::InclusiveSum),
// :70-111 (duplicateWithKeys), :35-50 + :381-386 (getHigherMsb +
// cub::DeviceRadixSort::SortPairs on bits [0, 32+bit)), :173-195 + :388
// (identifyTileRanges after a memset), with CR = submodules/
// diff-surfel-rasterization/cuda_rasterizer.  The sorted keys and values are
// produced by a depth sort of the splats followed by a tile-bits sort of the
// pairs (the last section below explains why the order is the same).
//
// Sort design (gfx950, 64-lane waves): reduce-then-scan LSD radix with 8-bit
// digits, three launches per pass.  Each 256-thread block owns 4096 keys
// (1024 for sorts of up to 4M keys, so that the splats' depth sort fills the
// chip); the histogram counts them with LDS atomics; one workgroup per digit
// scans that digit's block counts; the scatter's waves rank their keys in
// rounds of 64 with eight ballots per round (multi-split by digit), keeping
// the per-wave digit counters in LDS, which gives a stable rank without LDS
// atomics.  No kernel waits on another block, so there is no inter-block spin.
#include "nest_internal.h"
#include "nest_math.h"

namespace nest {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;  // 4096
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// block scan helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t wave_inclusive_scan_u64(uint64_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint64_t o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}

// Exclusive scan of one value per thread over a 256-thread block; returns
// the exclusive prefix and writes the block total to *total.
__device__ __forceinline__ uint64_t block_exclusive_scan_u64(uint64_t v, uint64_t* total) {
  __shared__ uint64_t wsum[kScanThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const uint64_t inc = wave_inclusive_scan_u64(v);
  if (lane == kWave - 1) wsum[wid] = inc;
  __syncthreads();
  uint64_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kScanThreads / kWave; w++) {
    const uint64_t s = wsum[w];
    if (w < wid) before += s;
    all += s;
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

// Pass 1: per-block totals (64-bit so an overflowing u32 total is detected).
__global__ void __launch_bounds__(kScanThreads) scan_reduce_kernel(const uint32_t* __restrict__ in, int64_t n,
                                                                  uint64_t* __restrict__ partial) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  uint64_t s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; k++) {
    const int64_t i = base + (int64_t)k * kScanThreads + threadIdx.x;
    if (i < n) s += in[i];
  }
  uint64_t total;
  block_exclusive_scan_u64(s, &total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// Pass 2: exclusive scan of the block totals in place, one block.  partial
// has nb entries; partial[nb] receives the grand total.
__global__ void __launch_bounds__(kScanThreads) scan_partials_kernel(uint64_t* __restrict__ partial, int64_t nb) {
  const int64_t per = (nb + kScanThreads - 1) / kScanThreads;
  const int64_t lo = (int64_t)threadIdx.x * per;
  const int64_t hi = lo + per < nb ? lo + per : nb;
  uint64_t s = 0;
  for (int64_t i = lo; i < hi; i++) s += partial[i];
  uint64_t total;
  uint64_t run = block_exclusive_scan_u64(s, &total);
  for (int64_t i = lo; i < hi; i++) {
    const uint64_t v = partial[i];
    partial[i] = run;
    run += v;
  }
  if (threadIdx.x == 0) partial[nb] = total;
}

// LDS index with one pad word per 16, so that lane t reading its 16
// consecutive items (stride 17 words) hits distinct banks.
__device__ __forceinline__ int padded(int i) { return i + (i >> 4); }

// Up to this many blocks, pass 3 sums the block totals before it itself (at
// most 4 loads per thread) and pass 2 is not launched.
constexpr int64_t kScanFoldBlocks = 1024;

// Pass 3: rescan each tile of 4096 items with its block offset.  Items are
// loaded coalesced (item k*256 + t), transposed through LDS so that each
// thread scans 16 consecutive items, and stored coalesced again.  kFold:
// partial holds the nb block totals unscanned; each block adds up those
// before it, and the last block writes the grand total to partial[nb].
template <bool kExclusive, bool kFold>
__global__ void __launch_bounds__(kScanThreads) scan_down_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                                int64_t n, uint64_t* __restrict__ partial) {
  __shared__ uint32_t tile[kScanTile + kScanTile / 16];
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  uint64_t before = 0;
  if constexpr (kFold) {
    for (uint32_t j = threadIdx.x; j < blockIdx.x; j += kScanThreads) before += partial[j];
  }
#pragma unroll
  for (int k = 0; k < kScanItems; k++) {
    const int idx = k * kScanThreads + threadIdx.x;
    const int64_t i = base + idx;
    tile[padded(idx)] = i < n ? in[i] : 0u;
  }
  __syncthreads();
  uint32_t v[kScanItems];
  uint64_t s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; k++) {
    v[k] = tile[padded(threadIdx.x * kScanItems + k)];
    s += v[k];
  }
  uint64_t total;
  uint64_t run = block_exclusive_scan_u64(s, &total);
  if constexpr (kFold) {
    uint64_t off;
    block_exclusive_scan_u64(before, &off);
    run += off;
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) partial[gridDim.x] = off + total;
  } else {
    run += partial[blockIdx.x];
  }
#pragma unroll
  for (int k = 0; k < kScanItems; k++) {
    if (kExclusive) {
      tile[padded(threadIdx.x * kScanItems + k)] = (uint32_t)run;
      run += v[k];
    } else {
      run += v[k];
      tile[padded(threadIdx.x * kScanItems + k)] = (uint32_t)run;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kScanItems; k++) {
    const int idx = k * kScanThreads + threadIdx.x;
    const int64_t i = base + idx;
    if (i < n) out[i] = tile[padded(idx)];
  }
}

size_t scan_ws_bytes(int64_t n) {
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  return (size_t)(nb + 1) * sizeof(uint64_t);
}

static hipError_t scan_impl(const uint32_t* in, uint32_t* out, int64_t n, void* ws, bool exclusive, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  uint64_t* partial = static_cast<uint64_t*>(ws);
  hipLaunchKernelGGL(scan_reduce_kernel, dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, n, partial);
  if (nb <= kScanFoldBlocks) {
    if (exclusive)
      hipLaunchKernelGGL((scan_down_kernel<true, true>), dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, out, n,
                         partial);
    else
      hipLaunchKernelGGL((scan_down_kernel<false, true>), dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, out, n,
                         partial);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanThreads), 0, s, partial, nb);
  if (exclusive)
    hipLaunchKernelGGL((scan_down_kernel<true, false>), dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, out, n,
                       partial);
  else
    hipLaunchKernelGGL((scan_down_kernel<false, false>), dim3((unsigned)nb), dim3(kScanThreads), 0, s, in, out, n,
                       partial);
  return hipGetLastError();
}

hipError_t launch_scan_u32(const uint32_t* in, uint32_t* out, int64_t n, void* ws, hipStream_t s) {
  return scan_impl(in, out, n, ws, false, s);
}

// ---------------------------------------------------------------------------
// fill, duplicate, ranges
// ---------------------------------------------------------------------------

__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t value, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = value;
}

hipError_t launch_fill_u32(uint32_t* dst, uint32_t value, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, value, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// radix sort
// ---------------------------------------------------------------------------

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;                          // rounds of 64 keys per wave (large sorts)
constexpr int kSortRoundsSmall = 4;                      // up to kSmallSort keys: 1024 keys per block
constexpr int64_t kSmallSort = 1 << 22;
constexpr int kSortWaves = kSortThreads / kWave;         // 4

// Lanes of the calling wave whose 8-bit digit equals d, restricted to 'valid'.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t valid) {
  uint64_t peers = valid;
#pragma unroll
  for (int b = 0; b < kRadixBits; b++) {
    const uint64_t m = __ballot((d >> b) & 1u);
    peers &= ((d >> b) & 1u) ? m : ~m;
  }
  return peers;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & (kWave - 1);
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Per-block digit histogram, written digit-major: counts[d * nblocks + b].
// The block's keys are counted with LDS atomics (a count does not depend on
// the order in which they land).
template <typename K, int R>
__global__ void __launch_bounds__(kSortThreads) radix_hist_kernel(const K* __restrict__ keys, int64_t n, int shift,
                                                                 int nbits, uint32_t* __restrict__ counts,
                                                                 uint32_t nblocks) {
  const uint32_t dmask = (1u << nbits) - 1u;
  __shared__ uint32_t hist[kRadix];
  for (int i = threadIdx.x; i < kRadix; i += kSortThreads) hist[i] = 0;
  const int64_t base = (int64_t)blockIdx.x * (kSortThreads * R);
  // all of the thread's keys in flight at once
  K key[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t i = base + r * kSortThreads + threadIdx.x;
    key[r] = i < n ? keys[i] : (K)0;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t i = base + r * kSortThreads + threadIdx.x;
    if (i < n) atomicAdd(&hist[(uint32_t)(key[r] >> shift) & dmask], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < kRadix; d += kSortThreads) counts[(size_t)d * nblocks + blockIdx.x] = hist[d];
}

// Exclusive scan of each digit's block counts in place, one workgroup per
// digit (counts[d * nb + b] becomes the count of digit d in the blocks before
// b); dtot[d] receives the digit's total.  The scatter adds the digits'
// exclusive prefix: together that is the exclusive scan of the digit-major
// counts.  The launch also zeroes zero[0, nzero) (the per-tile counters of
// the tile sort's last pass), since it runs right before that pass.
constexpr int kDigitHeld = 16;  // block counts per thread held in registers (up to 4096 blocks)

__global__ void __launch_bounds__(kScanThreads) digit_scan_kernel(uint32_t* __restrict__ counts, uint32_t nb,
                                                                 uint32_t* __restrict__ dtot, uint32_t* __restrict__ zero,
                                                                 uint32_t nzero) {
  uint32_t* c = counts + (size_t)blockIdx.x * nb;
  const uint32_t per = (nb + kScanThreads - 1) / kScanThreads;
  const uint32_t lo = threadIdx.x * per, hi = min(lo + per, nb);
  // the thread's first kDigitHeld counts: loads all in flight at once (a loop
  // with a runtime trip count issues them one by one), kept for the rewrite
  uint32_t v[kDigitHeld];
#pragma unroll
  for (int k = 0; k < kDigitHeld; k++) v[k] = lo + k < hi ? c[lo + k] : 0u;
  uint64_t s = 0;
#pragma unroll
  for (int k = 0; k < kDigitHeld; k++) s += v[k];
  for (uint32_t i = lo + kDigitHeld; i < hi; i++) s += c[i];
  uint64_t total;
  uint64_t run = block_exclusive_scan_u64(s, &total);
#pragma unroll
  for (int k = 0; k < kDigitHeld; k++) {
    if (lo + k < hi) {
      c[lo + k] = (uint32_t)run;
      run += v[k];
    }
  }
  for (uint32_t i = lo + kDigitHeld; i < hi; i++) {
    const uint32_t x = c[i];
    c[i] = (uint32_t)run;
    run += x;
  }
  if (threadIdx.x == 0) dtot[blockIdx.x] = (uint32_t)total;
  for (uint32_t i = blockIdx.x * kScanThreads + threadIdx.x; i < nzero; i += gridDim.x * kScanThreads) zero[i] = 0u;
}

// Stable scatter of one digit pass.  offsets[d * nb + b] is the count of
// digit d in the blocks before b and dtot[d] the digit's total.  The block's
// keys are first placed in LDS in digit order (stable), then written out so
// that consecutive lanes write consecutive positions of each digit's run.
// KOut == uint64_t with K == uint32_t composes the output key as
// (key << 32) | low_bits[val] (the tile/depth key of the binning stage);
// keys_out NULL writes the values alone.
// With tile_counts (the last pass of the tile sort, where a block's LDS copy
// is sorted on the whole key), every run of equal keys in that copy adds its
// length to tile_counts[2 * key + 1] (the .y of the key's uint2 range); keys
// at or past ntiles are not counted.
// With rect_in (the last pass of the splats' depth sort), each value v also
// carries its tile rectangle rect_in[v] to rect_out and the rectangle's tile
// count to area_out, at the value's sorted position.
template <typename K, typename KOut, int R>
__global__ void __launch_bounds__(kSortThreads) radix_scatter_kernel(const K* __restrict__ keys_in,
                                                                    const uint32_t* __restrict__ vals_in,
                                                                    KOut* __restrict__ keys_out,
                                                                    uint32_t* __restrict__ vals_out, int64_t n, int shift,
                                                                    int nbits,
                                                                    const uint32_t* __restrict__ offsets, uint32_t nblocks,
                                                                    const uint32_t* __restrict__ dtot,
                                                                    const uint32_t* __restrict__ low_bits,
                                                                    uint32_t* __restrict__ tile_counts, uint32_t ntiles,
                                                                    const uint2* __restrict__ rect_in,
                                                                    uint2* __restrict__ rect_out,
                                                                    uint32_t* __restrict__ area_out) {
  static_assert(kRadix == kSortThreads, "one digit per thread in the block scan");
  __shared__ uint32_t hist[kSortWaves][kRadix];
  __shared__ uint32_t gbase[kRadix];  // global start of the digit's run, minus its local start
  __shared__ K skey[kSortThreads * R];
  __shared__ uint32_t sval[kSortThreads * R];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const uint32_t dmask = (1u << nbits) - 1u;
  // the keys and values are in flight together with the digit offsets
  const int64_t base = (int64_t)blockIdx.x * (kSortThreads * R) + (int64_t)wid * (kWave * R);
  K key[R];
  uint32_t val[R];
  uint32_t rank[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t i = base + r * kWave + lane;
    if (i < n) {
      key[r] = keys_in[i];
      val[r] = vals_in ? vals_in[i] : (uint32_t)i;
    } else {
      key[r] = 0;
      val[r] = 0;
    }
  }
  for (int i = threadIdx.x; i < kSortWaves * kRadix; i += kSortThreads) (&hist[0][0])[i] = 0;
  {
    // thread d: the digit's global start, the exclusive prefix of the totals
    const int d = threadIdx.x;
    uint64_t all;
    const uint64_t dstart = block_exclusive_scan_u64(dtot[d], &all);
    gbase[d] = (uint32_t)dstart + offsets[(size_t)d * nblocks + blockIdx.x];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t i = base + r * kWave + lane;
    const bool ok = i < n;
    const uint32_t d = (uint32_t)(key[r] >> shift) & dmask;
    const uint64_t valid = __ballot(ok);
    const uint64_t peers = match_digit(d, valid);
    uint32_t before = 0;
    if (ok) before = hist[wid][d];
    rank[r] = before + (uint32_t)__popcll(peers & lanemask_lt());
    const int leader = __ffsll((unsigned long long)peers) - 1;
    if (ok && lane == leader) hist[wid][d] = before + (uint32_t)__popcll(peers);
  }
  __syncthreads();
  // thread d: wave-exclusive prefix of digit d, then the block-exclusive
  // prefix over digits (the digit's local start)
  {
    const int d = threadIdx.x;
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; w++) {
      const uint32_t c = hist[w][d];
      hist[w][d] = run;
      run += c;
    }
    uint64_t total;
    const uint32_t lstart = (uint32_t)block_exclusive_scan_u64(run, &total);
#pragma unroll
    for (int w = 0; w < kSortWaves; w++) hist[w][d] += lstart;
    gbase[d] -= lstart;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t i = base + r * kWave + lane;
    if (i < n) {
      const uint32_t d = (uint32_t)(key[r] >> shift) & dmask;
      const uint32_t lp = hist[wid][d] + rank[r];
      skey[lp] = key[r];
      sval[lp] = val[r];
    }
  }
  __syncthreads();
  const int64_t left = n - (int64_t)blockIdx.x * (kSortThreads * R);
  const int count = left < kSortThreads * R ? (int)left : kSortThreads * R;
  for (int j = threadIdx.x; j < count; j += kSortThreads) {
    const K k = skey[j];
    const uint32_t v = sval[j];
    const uint32_t pos = gbase[(uint32_t)(k >> shift) & dmask] + (uint32_t)j;
    // keys_out NULL (the tile sort's last pass in the forward): the values
    // alone, no depth-bits gather and no key write
    if (keys_out != nullptr) {
      if constexpr (sizeof(KOut) > sizeof(K))
        keys_out[pos] = ((KOut)k << 32) | (KOut)low_bits[v];
      else
        keys_out[pos] = k;
    }
    vals_out[pos] = v;
    if (rect_in != nullptr) {
      const uint2 rc = rect_in[v];
      rect_out[pos] = rc;
      area_out[pos] = ((rc.y & 0xFFFFu) - (rc.x & 0xFFFFu)) * ((rc.y >> 16) - (rc.x >> 16));
    }
    if (tile_counts != nullptr && (uint64_t)k < ntiles) {
      // the run [a, b) of key k adds -a at its first element, b at its last
      uint32_t* c = tile_counts + 2u * (uint32_t)k + 1u;
      if (j == 0 || skey[j - 1] != k) atomicSub(c, (uint32_t)j);
      if (j == count - 1 || skey[j + 1] != k) atomicAdd(c, (uint32_t)(j + 1));
    }
  }
}

// Tile ranges from the per-tile pair counts of the sorted pairs, one
// workgroup: ranges[t] = [start, start + count) with start the exclusive scan
// of the counts, and (0, 0) for a tile without pairs, as identifyTileRanges
// leaves it after the memset.  The counts are read from ranges[t].y (the tile
// sort's last pass accumulates them there, x zero) and overwritten in place.
constexpr int kRangeThreads = 1024;
constexpr uint32_t kRangeLds = 16384;  // counts staged in LDS up to this many tiles

__global__ void __launch_bounds__(kRangeThreads) ranges_from_counts_kernel(uint2* __restrict__ ranges,
                                                                          uint32_t ntiles) {
  __shared__ uint32_t wsum[kRangeThreads / kWave];
  __shared__ uint32_t cnt[kRangeLds];
  const uint32_t per = (ntiles + kRangeThreads - 1) / kRangeThreads;
  const uint32_t lo = threadIdx.x * per, hi = min(lo + per, ntiles);
  const bool staged = ntiles <= kRangeLds;
  if (staged) {
    // all counts in flight at once (coalesced, a fixed count per thread), then
    // each thread's run from LDS
    static_assert(kRangeLds % kRangeThreads == 0, "whole rounds of loads");
    uint32_t v[kRangeLds / kRangeThreads];
#pragma unroll
    for (int k = 0; k < (int)(kRangeLds / kRangeThreads); k++) {
      const uint32_t t = threadIdx.x + (uint32_t)k * kRangeThreads;
      v[k] = t < ntiles ? ranges[t].y : 0u;
    }
#pragma unroll
    for (int k = 0; k < (int)(kRangeLds / kRangeThreads); k++) {
      const uint32_t t = threadIdx.x + (uint32_t)k * kRangeThreads;
      if (t < ntiles) cnt[t] = v[k];
    }
    __syncthreads();
  }
  uint32_t s = 0;
  for (uint32_t t = lo; t < hi; t++) s += staged ? cnt[t] : ranges[t].y;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  uint32_t inc = s;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += o;
  }
  if (lane == kWave - 1) wsum[wid] = inc;
  __syncthreads();
  uint32_t run = inc - s;
  for (int w = 0; w < wid; w++) run += wsum[w];
  if (staged) {
    // each run start replaces its count in LDS; the ranges go out coalesced
    for (uint32_t t = lo; t < hi; t++) {
      const uint32_t c = cnt[t];
      cnt[t] = run;
      run += c;
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < ntiles; t += kRangeThreads) {
      const uint32_t st = cnt[t];
      const uint32_t en = t + 1 < ntiles ? cnt[t + 1] : st + ranges[t].y;
      ranges[t] = en != st ? make_uint2(st, en) : make_uint2(0u, 0u);
    }
    return;
  }
  for (uint32_t t = lo; t < hi; t++) {
    const uint32_t c = ranges[t].y;
    ranges[t] = c != 0u ? make_uint2(run, run + c) : make_uint2(0u, 0u);
    run += c;
  }
}

// Keys per block: 1024 up to kSmallSort keys (more blocks to fill the chip for
// the splats' depth sort), else 4096 (longer runs per digit in the output;
// 8192 keys, 69 KB of LDS and 2 waves per SIMD, made the tile passes slower).
static int sort_rounds(int64_t n) { return n <= kSmallSort ? kSortRoundsSmall : kSortRounds; }
static int64_t sort_blocks(int64_t n) {
  const int64_t tile = (int64_t)kSortThreads * sort_rounds(n);
  return (n + tile - 1) / tile;
}
static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace: ping-pong keys/vals (two sets when the last pass widens the
// key), digit counts and their scan.
template <typename K, typename KOut>
static size_t sort_ws_bytes_t(int64_t n) {
  constexpr int sets = sizeof(KOut) == sizeof(K) ? 1 : 2;
  const int64_t ncounts = (int64_t)kRadix * sort_blocks(n);
  return sets * (align256((size_t)n * sizeof(K)) + align256((size_t)n * 4)) + align256((size_t)ncounts * 4) +
         align256((size_t)kRadix * 4);
}

// Stable LSD sort of (keys_in, vals_in) on key bits [0, end_bit) into
// (keys_out, vals_out).  The inputs are never written.  vals_in == nullptr
// stands for vals_in[i] = i.  With KOut wider than K the last pass writes
// (key << 32) | low_bits[val].  With tile_counts (ntiles uint2 ranges), the
// last pass also counts the keys per value (the pairs per tile) into the .y
// words, after zeroing all 2 * ntiles words.  With rect_in, the last pass
// writes no keys; it moves each value's rectangle and tile count to
// rect_out / area_out instead (area_out must not alias keys_in unless there
// is more than one pass).
template <typename K, typename KOut>
static hipError_t sort_impl(const K* keys_in, const uint32_t* vals_in, KOut* keys_out, uint32_t* vals_out, int64_t n,
                            int end_bit, const uint32_t* low_bits, void* ws, hipStream_t s,
                            uint32_t* tile_counts = nullptr, uint32_t ntiles = 0, const uint2* rect_in = nullptr,
                            uint2* rect_out = nullptr, uint32_t* area_out = nullptr) {
  if (n <= 0) return hipSuccess;
  constexpr bool kSame = sizeof(KOut) == sizeof(K);
  const int64_t nb = sort_blocks(n);
  const bool small = sort_rounds(n) == kSortRoundsSmall;
  const int64_t ncounts = (int64_t)kRadix * nb;
  char* w = static_cast<char*>(ws);
  K* tk[2];
  uint32_t* tv[2];
  for (int t = 0; t < (kSame ? 1 : 2); t++) {
    tk[t] = reinterpret_cast<K*>(w);
    w += align256((size_t)n * sizeof(K));
    tv[t] = reinterpret_cast<uint32_t*>(w);
    w += align256((size_t)n * 4);
  }
  uint32_t* counts = reinterpret_cast<uint32_t*>(w);
  w += align256((size_t)ncounts * 4);
  uint32_t* dtot = reinterpret_cast<uint32_t*>(w);

  int passes = (end_bit + kRadixBits - 1) / kRadixBits;
  if (passes < 1) passes = 1;
  const K* sk = keys_in;
  const uint32_t* sv = vals_in;
  for (int pass = 0; pass < passes; pass++) {
    const bool last = pass == passes - 1;
    const int shift = pass * kRadixBits;
    // bits of this pass's digit below end_bit (the sort ignores the bits above)
    const int nbits = end_bit - shift < kRadixBits ? (end_bit - shift > 0 ? end_bit - shift : 1) : kRadixBits;
    if (small)
      hipLaunchKernelGGL((radix_hist_kernel<K, kSortRoundsSmall>), dim3((unsigned)nb), dim3(kSortThreads), 0, s, sk, n,
                         shift, nbits, counts, (uint32_t)nb);
    else
      hipLaunchKernelGGL((radix_hist_kernel<K, kSortRounds>), dim3((unsigned)nb), dim3(kSortThreads), 0, s, sk, n,
                         shift, nbits, counts, (uint32_t)nb);
    uint32_t* tc = last ? tile_counts : nullptr;
    hipLaunchKernelGGL(digit_scan_kernel, dim3(kRadix), dim3(kScanThreads), 0, s, counts, (uint32_t)nb, dtot, tc,
                       tc ? 2u * ntiles : 0u);
    K* dk;
    uint32_t* dv;
    if constexpr (kSame) {
      // alternate so that the last pass lands in *_out
      const bool to_out = ((passes - 1 - pass) % 2) == 0;
      dk = to_out ? reinterpret_cast<K*>(keys_out) : tk[0];
      dv = to_out ? vals_out : tv[0];
    } else {
      dk = tk[pass & 1];
      dv = tv[pass & 1];
    }
    const uint2* ri = last ? rect_in : nullptr;
    uint2* ro = last ? rect_out : nullptr;
    uint32_t* ao = last ? area_out : nullptr;
    if (!kSame && last) {
      if (small)
        hipLaunchKernelGGL((radix_scatter_kernel<K, KOut, kSortRoundsSmall>), dim3((unsigned)nb), dim3(kSortThreads), 0,
                           s, sk, sv, keys_out, vals_out, n, shift, nbits, counts, (uint32_t)nb, dtot, low_bits, tc, ntiles,
                           ri, ro, ao);
      else
        hipLaunchKernelGGL((radix_scatter_kernel<K, KOut, kSortRounds>), dim3((unsigned)nb), dim3(kSortThreads), 0, s,
                           sk, sv, keys_out, vals_out, n, shift, nbits, counts, (uint32_t)nb, dtot, low_bits, tc, ntiles,
                           ri, ro, ao);
    } else {
      K* dko = ri != nullptr ? nullptr : dk;  // the rectangles replace the sorted keys
      if (small)
        hipLaunchKernelGGL((radix_scatter_kernel<K, K, kSortRoundsSmall>), dim3((unsigned)nb), dim3(kSortThreads), 0, s,
                           sk, sv, dko, dv, n, shift, nbits, counts, (uint32_t)nb, dtot, low_bits, tc, ntiles, ri, ro,
                           ao);
      else
        hipLaunchKernelGGL((radix_scatter_kernel<K, K, kSortRounds>), dim3((unsigned)nb), dim3(kSortThreads), 0, s, sk,
                           sv, dko, dv, n, shift, nbits, counts, (uint32_t)nb, dtot, low_bits, tc, ntiles, ri, ro, ao);
    }
    sk = dk;
    sv = dv;
  }
  return hipGetLastError();
}

size_t sort_ws_bytes(int64_t n) { return sort_ws_bytes_t<uint64_t, uint64_t>(n); }

hipError_t launch_sort_pairs(const uint64_t* keys_in, const uint32_t* vals_in, uint64_t* keys_out, uint32_t* vals_out,
                             int64_t n, int end_bit, void* ws, hipStream_t s) {
  return sort_impl<uint64_t, uint64_t>(keys_in, vals_in, keys_out, vals_out, n, end_bit, nullptr, ws, s);
}

// ---------------------------------------------------------------------------
// binning in depth order
// ---------------------------------------------------------------------------
//
// The reference sorts every (tile << 32 | depth bits, splat) pair on all
// 32 + tile bits.  Sorting the splats by depth first (stable, so equal depths
// keep splat order), emitting each splat's pairs in that order and then
// stable-sorting the pairs on the tile bits alone yields the same order:
// within a tile, by depth bits, then by splat index, which is where the
// reference's stable sort of the splat-ordered pairs puts equal keys.  The
// pair sort then runs on 4-byte keys over ceil(tile bits / 8) passes instead
// of 8-byte keys over ceil((32 + tile bits) / 8) passes.

size_t depth_order_ws_bytes(int P) {
  const int64_t n = P > 0 ? P : 1;
  return align256((size_t)n * 4) * 2 + sort_ws_bytes_t<uint32_t, uint32_t>(n);
}

// The depth keys (depth bits of the visible splats, whose depth is > 0.2 so
// that the bit order is the float order; 0xffffffff for culled splats, which
// emit no pairs and go last) are written by preprocess at the start of ws.
hipError_t launch_depth_order(int P, const uint32_t* rect, uint32_t* order, uint32_t* ordered_offsets,
                              uint32_t* ordered_rect, void* ws, hipStream_t s) {
  if (P <= 0) return hipSuccess;
  char* w = static_cast<char*>(ws);
  uint32_t* keys = reinterpret_cast<uint32_t*>(w);
  w += align256((size_t)P * 4);
  uint32_t* keys_sorted = reinterpret_cast<uint32_t*>(w);
  w += align256((size_t)P * 4);
  // 4 passes: the depth keys are read by the first alone, so the last pass
  // writes the tiles touched in depth order over them, next to the rectangles
  hipError_t e = sort_impl<uint32_t, uint32_t>(keys, nullptr, keys_sorted, order, P, 32, nullptr, w, s, nullptr, 0,
                                               reinterpret_cast<const uint2*>(rect),
                                               reinterpret_cast<uint2*>(ordered_rect), keys);
  if (e != hipSuccess) return e;
  // tiles touched in depth order, scanned (exclusive); the sort's workspace
  // is free again and holds the scan partials
  return scan_impl(keys, ordered_offsets, P, w, true, s);
}

// A workgroup owns 256 consecutive splats of the depth order, whose pairs
// form one contiguous run of the output.  Each splat's (offset, id, tile
// rectangle, read in depth order) goes to LDS; lanes then write consecutive pair positions
// (coalesced), each finding its splat by binary search over the offsets.
// Pair q of a splat is tile (y0 + q / w, x0 + q % w): row-major over the
// rectangle, as the reference emits them.  Writes stop at n_pairs (the pair
// buffers' length), whatever count the caller passed.
constexpr int kDupThreads = 256;

__global__ void __launch_bounds__(kDupThreads) duplicate_ordered_kernel(int P, const uint32_t* __restrict__ order,
                                                                       const uint32_t* __restrict__ offsets,
                                                                       const uint2* __restrict__ rect, uint32_t gx,
                                                                       uint32_t n_pairs,
                                                                       uint32_t* __restrict__ tile_keys,
                                                                       uint32_t* __restrict__ ids) {
  __shared__ uint32_t s_off[kDupThreads], s_id[kDupThreads], s_x0[kDupThreads], s_y0[kDupThreads], s_w[kDupThreads];
  const int k0 = blockIdx.x * kDupThreads;
  const int k = k0 + (int)threadIdx.x;
  // end of this group's run: the next group's first offset, or the total
  const uint32_t end = (k0 + kDupThreads < P) ? offsets[k0 + kDupThreads] : n_pairs;
  uint32_t off = end, id = 0, x0 = 0, y0 = 0, w = 1;
  if (k < P) {
    off = offsets[k];
    id = order[k];
    // culled splats have an empty rectangle and no pairs
    const uint2 rc = rect[k];
    x0 = rc.x & 0xFFFFu;
    y0 = rc.x >> 16;
    const uint32_t x1 = rc.y & 0xFFFFu;
    w = x1 > x0 ? x1 - x0 : 1u;
  }
  s_off[threadIdx.x] = off;
  s_id[threadIdx.x] = id;
  s_x0[threadIdx.x] = x0;
  s_y0[threadIdx.x] = y0;
  s_w[threadIdx.x] = w;
  __syncthreads();
  const uint32_t begin = s_off[0];
  const uint32_t stop = end < n_pairs ? end : n_pairs;
  for (uint32_t p = begin + threadIdx.x; p < stop; p += kDupThreads) {
    // last splat s with s_off[s] <= p; splats without pairs share their
    // offset with the next one and are never chosen
    int s = 0;
#pragma unroll
    for (int step = kDupThreads / 2; step > 0; step >>= 1)
      if (s_off[s + step] <= p) s += step;
    const uint32_t q = p - s_off[s];
    const uint32_t ws = s_w[s];
    const uint32_t dy = q / ws;
    tile_keys[p] = (s_y0[s] + dy) * gx + s_x0[s] + (q - dy * ws);
    ids[p] = s_id[s];
  }
}

hipError_t launch_duplicate_ordered(int P, const uint32_t* order, const uint32_t* offsets, const uint32_t* ordered_rect,
                                    uint32_t gx, int64_t n_pairs, uint32_t* tile_keys, uint32_t* ids, hipStream_t s) {
  if (P <= 0 || n_pairs <= 0) return hipSuccess;
  hipLaunchKernelGGL(duplicate_ordered_kernel, dim3((P + kDupThreads - 1) / kDupThreads), dim3(kDupThreads), 0, s, P,
                     order, offsets, reinterpret_cast<const uint2*>(ordered_rect), gx, (uint32_t)n_pairs, tile_keys,
                     ids);
  return hipGetLastError();
}

size_t tile_sort_ws_bytes(int64_t n) { return sort_ws_bytes_t<uint32_t, uint64_t>(n); }

hipError_t launch_sort_tiles(const uint32_t* tile_keys, const uint32_t* ids, uint64_t* keys_out, uint32_t* vals_out,
                             int64_t n, int tile_bits, const float* depth, uint32_t* ranges, uint32_t ntiles, void* ws,
                             hipStream_t s) {
  return sort_impl<uint32_t, uint64_t>(tile_keys, ids, keys_out, vals_out, n, tile_bits,
                                       reinterpret_cast<const uint32_t*>(depth), ws, s, ranges, ntiles);
}

// The reference's sorted keys, tile << 32 | depth bits of the pair's splat
// (point_list_keys, CR/rasterizer_impl.cu:381-386), from the tile ranges and
// the sorted point list: one workgroup per tile, its positions in order.
__global__ void __launch_bounds__(256) compose_keys_kernel(const uint2* __restrict__ ranges,
                                                            const uint32_t* __restrict__ point_list,
                                                            const uint32_t* __restrict__ depth_bits,
                                                            uint64_t* __restrict__ keys) {
  const uint32_t t = blockIdx.x;
  const uint2 r = ranges[t];
  for (uint32_t i = r.x + threadIdx.x; i < r.y; i += 256u) keys[i] = ((uint64_t)t << 32) | depth_bits[point_list[i]];
}

hipError_t launch_compose_keys(const uint32_t* ranges, const uint32_t* point_list, const float* depth, uint32_t ntiles,
                               uint64_t* keys, hipStream_t s) {
  if (ntiles == 0) return hipSuccess;
  hipLaunchKernelGGL(compose_keys_kernel, dim3(ntiles), dim3(256), 0, s, reinterpret_cast<const uint2*>(ranges),
                     point_list, reinterpret_cast<const uint32_t*>(depth), keys);
  return hipGetLastError();
}

// identifyTileRanges: with pairs, turns the per-tile counts that
// launch_sort_tiles left in ranges into [start, end) ranges; without pairs,
// zeroes the ranges.
hipError_t launch_tile_ranges(uint32_t* ranges, int64_t n, uint32_t ntiles, hipStream_t s) {
  if (n <= 0 || ntiles == 0) return launch_fill_u32(ranges, 0u, 2 * (int64_t)ntiles, s);
  hipLaunchKernelGGL(ranges_from_counts_kernel, dim3(1), dim3(kRangeThreads), 0, s, reinterpret_cast<uint2*>(ranges),
                     ntiles);
  return hipGetLastError();
}

}  // namespace nest
