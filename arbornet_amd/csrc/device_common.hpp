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

// ---------------------------------------------------------------------------------------
// Cross-lane primitives without LDS: DPP moves inside rows of 16 lanes and the gfx950
// permlane swaps across rows (v_permlane16_swap / v_permlane32_swap). All of them expect
// every lane of the wave to be active.
// ---------------------------------------------------------------------------------------
template <typename T, typename F>
__device__ __forceinline__ T map_dwords(T v, F f) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  uint32_t d[sizeof(T) / 4];
  __builtin_memcpy(d, &v, sizeof(T));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) d[i] = f(d[i], i);
  T r;
  __builtin_memcpy(&r, d, sizeof(T));
  return r;
}

// DPP move: lanes whose source is outside the row (or whose row is masked off) get `old`.
template <int CTRL, int ROW_MASK = 0xF, typename T>
__device__ __forceinline__ T dpp_mov(T old, T v) {
  uint32_t o[sizeof(T) / 4];
  __builtin_memcpy(o, &old, sizeof(T));
  return map_dwords(v, [&](uint32_t x, int i) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)o[i], (int)x, CTRL, ROW_MASK, 0xF, false);
  });
}
constexpr int kDppQuadXor1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppQuadRev = 0x1B;     // quad_perm [3,2,1,0]
constexpr int kDppRowShr = 0x110;     // + n: row_shr:n
constexpr int kDppWaveShr1 = 0x138;   // wave_shr:1
constexpr int kDppRowMirror = 0x140;  // lane 15 - i within the row
constexpr int kDppHalfMirror = 0x141; // lane 7 - i within the half-row
constexpr int kDppBcast15 = 0x142;    // lane 15 of the row above
constexpr int kDppBcast31 = 0x143;    // lane 31

// lo[i] = v[i & ~S], hi[i] = v[i | S] for S = 16 (rows) or 32 (halves).
template <int S, typename T>
__device__ __forceinline__ void lane_split(T v, T& lo, T& hi) {
  uint32_t d[sizeof(T) / 4], l[sizeof(T) / 4], h[sizeof(T) / 4];
  __builtin_memcpy(d, &v, sizeof(T));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) {
    if constexpr (S == 16) {
      const auto p = __builtin_amdgcn_permlane16_swap(d[i], d[i], false, false);
      l[i] = p[0];
      h[i] = p[1];
    } else {
      const auto p = __builtin_amdgcn_permlane32_swap(d[i], d[i], false, false);
      l[i] = p[0];
      h[i] = p[1];
    }
  }
  __builtin_memcpy(&lo, l, sizeof(T));
  __builtin_memcpy(&hi, h, sizeof(T));
}

// Value of lane (lane ^ J), J a power of two <= 32.
template <int J, typename T>
__device__ __forceinline__ T lane_xor(T v) {
  if constexpr (J == 1) {
    return dpp_mov<kDppQuadXor1>(v, v);
  } else if constexpr (J == 2) {
    return dpp_mov<kDppQuadXor2>(v, v);
  } else if constexpr (J == 4) {
    return dpp_mov<kDppQuadRev>(v, dpp_mov<kDppHalfMirror>(v, v));  // (i ^ 7) ^ 3
  } else if constexpr (J == 8) {
    return dpp_mov<kDppHalfMirror>(v, dpp_mov<kDppRowMirror>(v, v));  // (i ^ 15) ^ 7
  } else {
    static_assert(J == 16 || J == 32, "power of two <= 32");
    T lo, hi;
    lane_split<J>(v, lo, hi);
    return (lane_id() & J) ? lo : hi;
  }
}
// lane_xor with a stride known only after unrolling
template <typename T>
__device__ __forceinline__ T lane_xor_n(T v, int j) {
  switch (j) {
    case 1: return lane_xor<1>(v);
    case 2: return lane_xor<2>(v);
    case 4: return lane_xor<4>(v);
    case 8: return lane_xor<8>(v);
    case 16: return lane_xor<16>(v);
    default: return lane_xor<32>(v);
  }
}
// Value of lane 63 - lane.
template <typename T>
__device__ __forceinline__ T lane_reverse(T v) {
  return lane_xor<32>(lane_xor<16>(dpp_mov<kDppRowMirror>(v, v)));
}
// A wave-uniform value, marked as such for the compiler (kept in a scalar register).
template <typename T>
__device__ __forceinline__ T uniform(T v) {
  static_assert(sizeof(T) == 4, "32-bit values");
  int i;
  __builtin_memcpy(&i, &v, 4);
  i = __builtin_amdgcn_readfirstlane(i);
  __builtin_memcpy(&v, &i, 4);
  return v;
}

// Value of lane `src` (wave-uniform) in every lane.
template <typename T>
__device__ __forceinline__ T lane_get(T v, int src) {
  return map_dwords(v, [&](uint32_t x, int) { return (uint32_t)__builtin_amdgcn_readlane((int)x, src); });
}
// Value of lane - 1 (lane 0 gets `fill`).
template <typename T>
__device__ __forceinline__ T lane_shift_down(T v, T fill) {
  return dpp_mov<kDppWaveShr1>(fill, v);
}

// Butterfly reduction; every lane gets the result, bitwise identical in every lane.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  v = op(v, lane_xor<1>(v));
  v = op(v, lane_xor<2>(v));
  v = op(v, dpp_mov<kDppHalfMirror>(v, v));
  v = op(v, dpp_mov<kDppRowMirror>(v, v));
  T lo, hi;
  lane_split<16>(v, lo, hi);
  v = op(lo, hi);
  lane_split<32>(v, lo, hi);
  return op(lo, hi);
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
  return wave_reduce(v, [](T x, T y) { return y > x ? y : x; });
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
  return wave_reduce(v, [](T x, T y) { return y < x ? y : x; });
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  return wave_reduce(v, [](T x, T y) { return x + y; });
}
// Inclusive prefix sum across the wave in lane order.
template <typename T>
__device__ __forceinline__ T wave_scan_incl(T v) {
  const T z = T(0);
  v = v + dpp_mov<kDppRowShr + 1>(z, v);
  v = v + dpp_mov<kDppRowShr + 2>(z, v);
  v = v + dpp_mov<kDppRowShr + 4>(z, v);
  v = v + dpp_mov<kDppRowShr + 8>(z, v);
  v = v + dpp_mov<kDppBcast15, 0xA>(z, v);
  v = v + dpp_mov<kDppBcast31, 0xC>(z, v);
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
  // at most one pass: the table has at least twice as many slots as ids, so a pass always
  // finds the id or a free slot; the bound only makes every probe finite
  for (uint32_t n = 0; n <= mask; ++n) {
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
  return false;
}

// Occurrence count of `id` (0 if absent).
__device__ __forceinline__ uint32_t hist_count(const uint32_t* tab, uint32_t bits, uint32_t id) {
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t s = hist_slot(id, bits);
  for (uint32_t n = 0; n <= mask; ++n) {  // at most one pass (see hist_insert)
    const uint32_t cur = tab[s];
    if (cur == kEmptySlot) return 0u;
    if ((cur >> 12) == id) return (cur & 4095u) + 1u;
    s = (s + 1u) & mask;
  }
  return 0u;
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
