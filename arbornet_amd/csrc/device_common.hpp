// device_common.hpp -- wave/block primitives and the per-element sampling math shared by
// the streaming kernel and the row solver (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

namespace arbor {

constexpr int kWave = 64;
constexpr uint32_t kEmptySlot = 0xFFFFFFFFu;  // empty history-table slot
constexpr uint32_t kKeyNegInf = 0x007FFFFFu;  // order_key(-inf)

// chunk / row status bits
constexpr uint32_t kFlagInvalid = 1u;     // NaN or +inf tempered logit
constexpr uint32_t kFlagBadHistory = 2u;  // history id >= vocab
constexpr uint32_t kFlagOverflow = 4u;    // candidate list did not fit: row goes to the row solver

// Fixed-point scale of probability mass in the row solver: q = e * 2^40, e in [0, 1].
// A row of at most 2^20 tokens sums to < 2^60, so the sums are exact in uint64 and do
// not depend on reduction order.
constexpr float kMassScale = 1099511627776.0f;  // 2^40

// Order-preserving key of a canonical (no -0) non-NaN float.
__device__ __forceinline__ uint32_t order_key(float z) {
  const uint32_t b = __float_as_uint(z);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// Composite rank key: larger = earlier in the ranking (z descending, then id ascending).
__device__ __forceinline__ uint64_t composite(float z, int32_t id) {
  return ((uint64_t)order_key(z) << 32) | (uint32_t)(~(uint32_t)id);
}
__device__ __forceinline__ int32_t composite_id(uint64_t c) { return (int32_t)(~(uint32_t)c); }
__device__ __forceinline__ float composite_z(uint64_t c) { return key_value((uint32_t)(c >> 32)); }

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Orders this wave's LDS accesses: every LDS op issued before completes before any after.
__device__ __forceinline__ void wave_lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Count of set bits of `mask` in lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                       __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const T w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const T w = __shfl_xor(v, o);
    v = w < v ? w : v;
  }
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
// Inclusive prefix sum across the wave in lane order.
template <typename T>
__device__ __forceinline__ T wave_scan_incl(T v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const T w = __shfl_up(v, o);
    if (lane >= o) v += w;
  }
  return v;
}

// ---------------------------------------------------------------------------------------
// History table: open addressing in LDS, entry = id << 12 | (count - 1), linear probing.
// ids < 2^20 and counts <= 4096 fit; the table holds at most half its slots.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hist_slot(uint32_t id, uint32_t bits) {
  return (id * 2654435761u) >> (32u - bits);
}

// Counts one occurrence of id; returns true for the call that created the entry.
__device__ __forceinline__ bool hist_insert(uint32_t* tab, uint32_t bits, uint32_t id) {
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t s = hist_slot(id, bits);
  for (;;) {
    uint32_t cur = tab[s];
    if (cur == kEmptySlot) {
      const uint32_t prev = atomicCAS(&tab[s], kEmptySlot, id << 12);
      if (prev == kEmptySlot) return true;
      cur = prev;
    }
    if ((cur >> 12) == id) {
      atomicAdd(&tab[s], 1u);
      return false;
    }
    s = (s + 1u) & mask;
  }
}

// Occurrence count of `id` (0 if absent).
__device__ __forceinline__ uint32_t hist_count(const uint32_t* tab, uint32_t bits, uint32_t id) {
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t s = hist_slot(id, bits);
  for (;;) {
    const uint32_t cur = tab[s];
    if (cur == kEmptySlot) return 0u;
    if ((cur >> 12) == id) return (cur & 4095u) + 1u;
    s = (s + 1u) & mask;
  }
}

struct Penalty {
  float rp, inv_rp, fp, pp;
};

// Repetition (once), then frequency * count + presence. One rounding per operation,
// the order of operations the contract fixes; the trailing + 0 turns -0 into +0.
__device__ __forceinline__ float penalize(float z, uint32_t count, const Penalty& p) {
  const float v = z > 0.0f ? z * p.inv_rp : z * p.rp;
  const float pen = (float)count * p.fp + p.pp;
  return (v - pen) + 0.0f;
}

// NaN or +inf
__device__ __forceinline__ bool is_invalid(float z) { return __builtin_amdgcn_classf(z, 1 | 2 | 512); }

__device__ __forceinline__ float bf16_bits_to_float(uint32_t h) { return __uint_as_float(h << 16); }

}  // namespace arbor
