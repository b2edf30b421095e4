// Block-level primitives for one-workgroup-per-row kernels (wave64, BLOCK
// lanes): exact 64-bit scans and sums, and the index-ordered inverse-CDF pick
// over a dense row whose weights are produced on the fly.
#pragma once

#include "ls_common.hpp"
#include "ls_numerics.hpp"

namespace ls {

__device__ __forceinline__ uint64_t wave_incl_scan64(uint64_t x, int lane) {
  (void)lane;
  return wave_scan_add_u64(x);
}

// Exclusive scan in lane order; *total receives the block sum. smem >= BLOCK/64.
template <int BLOCK>
__device__ __forceinline__ uint64_t block_excl_scan64(uint64_t v, uint64_t* smem, uint64_t* total) {
  constexpr int kWaves = BLOCK / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const uint64_t inc = wave_incl_scan64(v, lane);
  __syncthreads();
  if (lane == kWave - 1) smem[wid] = inc;
  __syncthreads();
  uint64_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const uint64_t s = smem[i];
    base += i < wid ? s : 0;
    tot += s;
  }
  *total = tot;
  return base + inc - v;
}

// Contiguous index range [a, b) of a row of n elements owned by this lane.
template <int BLOCK>
__device__ __forceinline__ void lane_range(int64_t n, int64_t* a, int64_t* b) {
  const int64_t per = (n + BLOCK - 1) / BLOCK;
  const int64_t s = static_cast<int64_t>(threadIdx.x) * per;
  *a = s < n ? s : n;
  *b = s + per < n ? s + per : n;
}

// Exact sum of fx46(w(i)) over the row (fewer than 128 terms per double
// accumulation keep every partial sum exact).
template <int BLOCK, typename W>
__device__ uint64_t row_mass(int64_t n, W w, uint64_t* smem) {
  int64_t a, b;
  lane_range<BLOCK>(n, &a, &b);
  uint64_t sum = 0;
  double acc = 0.0;
  int c = 0;
  for (int64_t i = a; i < b; ++i) {
    acc += fx46_d(w(i));
    if (++c == 100) {
      sum += static_cast<uint64_t>(acc);
      acc = 0.0;
      c = 0;
    }
  }
  sum += static_cast<uint64_t>(acc);
  return block_sum_u64<BLOCK>(sum, smem);
}

// First index j (index order) with sum_{i<=j} fx46(w(i)) > floor(u * total);
// index 0 when the total is zero (the reference's all-false argmax).
template <int BLOCK, typename W>
__device__ int64_t row_pick(int64_t n, float u, W w, uint64_t* smem, int64_t* result) {
  int64_t a, b;
  lane_range<BLOCK>(n, &a, &b);
  uint64_t sum = 0;
  double acc = 0.0;
  int c = 0;
  for (int64_t i = a; i < b; ++i) {
    acc += fx46_d(w(i));
    if (++c == 100) {
      sum += static_cast<uint64_t>(acc);
      acc = 0.0;
      c = 0;
    }
  }
  sum += static_cast<uint64_t>(acc);
  uint64_t total;
  const uint64_t ex = block_excl_scan64<BLOCK>(sum, smem, &total);
  if (threadIdx.x == 0) *result = 0;
  __syncthreads();
  if (total > 0) {
    const uint64_t target = floor_u_times(u, total);
    if (ex <= target && target < ex + sum) {
      uint64_t run = ex;
      for (int64_t i = a; i < b; ++i) {
        run += fx46(w(i));
        if (run > target) {
          *result = i;
          break;
        }
      }
    }
  }
  __syncthreads();
  return *result;
}

}  // namespace ls
