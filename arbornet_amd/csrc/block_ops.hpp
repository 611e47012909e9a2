// block_ops.hpp -- workgroup-level reductions, scans and sorts over LDS (gfx950, wave64).
#pragma once

#include "device_common.hpp"

namespace arbor {

template <int BLOCK, typename T>
__device__ T block_reduce_sum(T v, T* scratch) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (lane_id() == 0) scratch[w] = v;
  __syncthreads();
  T r = 0;
  for (int i = 0; i < BLOCK / kWave; ++i) r += scratch[i];
  __syncthreads();
  return r;
}

template <int BLOCK, typename T>
__device__ T block_reduce_max(T v, T* scratch) {
  v = wave_max(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (lane_id() == 0) scratch[w] = v;
  __syncthreads();
  T r = scratch[0];
  for (int i = 1; i < BLOCK / kWave; ++i) r = scratch[i] > r ? scratch[i] : r;
  __syncthreads();
  return r;
}

template <int BLOCK, typename T>
__device__ T block_reduce_min(T v, T* scratch) {
  v = wave_min(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (lane_id() == 0) scratch[w] = v;
  __syncthreads();
  T r = scratch[0];
  for (int i = 1; i < BLOCK / kWave; ++i) r = scratch[i] < r ? scratch[i] : r;
  __syncthreads();
  return r;
}

// Exclusive prefix sum across the block in thread order; *total gets the block sum.
template <int BLOCK, typename T>
__device__ __forceinline__ T block_scan_excl(T v, T* scratch, T* total) {
  const T incl = wave_scan_incl(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (lane_id() == kWave - 1) scratch[w] = incl;
  __syncthreads();
  T base = 0, tot = 0;
  for (int i = 0; i < BLOCK / kWave; ++i) {
    if (i < w) base += scratch[i];
    tot += scratch[i];
  }
  __syncthreads();
  *total = tot;
  return base + incl - v;
}

// Inclusive prefix sum of arr[0, n) in place, n <= BLOCK * ITEMS, arr in LDS.
template <int BLOCK, int ITEMS = 2>
__device__ void block_scan_array(double* arr, int n, double* scratch) {
  const int t = threadIdx.x;
  double loc[ITEMS];
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int i = t * ITEMS + j;
    s += i < n ? arr[i] : 0.0;
    loc[j] = s;
  }
  double tot;
  const double base = block_scan_excl<BLOCK, double>(s, scratch, &tot);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int i = t * ITEMS + j;
    if (i < n) arr[i] = base + loc[j];
  }
  __syncthreads();
}

// Ascending bitonic sort of arr[0, n) in LDS (arr has room for the next power of two).
template <int BLOCK>
__device__ void block_sort_asc(uint64_t* arr, int n) {
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = n + threadIdx.x; i < np; i += BLOCK) arr[i] = ~0ull;
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < np / 2; i += BLOCK) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool asc = (lo & size) == 0;
        const uint64_t x = arr[lo], y = arr[hi];
        if ((x > y) == asc) {
          arr[lo] = y;
          arr[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// Sort 64 values held one per lane, descending (bitonic network over DPP / permlane moves).
__device__ __forceinline__ uint64_t wave_sort64_desc(uint64_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t w = lane_xor_n(v, stride);
      const bool asc = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      const uint64_t mx = v > w ? v : w, mn = v > w ? w : v;
      v = (lower == asc) ? mx : mn;
    }
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_sort64_desc_u32(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t w = lane_xor_n(v, stride);
      const bool asc = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      const uint32_t mx = v > w ? v : w, mn = v > w ? w : v;
      v = (lower == asc) ? mx : mn;
    }
  }
  return v;
}

}  // namespace arbor
