// topk_path.hpp -- the streaming top-k path (1 <= k <= 64).
//
// Every wave keeps the 64 best candidates it has seen as a register-resident list: lane i
// holds the i-th best 64-bit rank key (order_key(z) << 32 | ~id; 0 = empty). Once the
// list holds k entries its k-th key is an exact threshold for everything the wave sees
// later, so after the first batch almost nothing passes it; what does pass is collected
// 64 at a time, sorted with a bitonic network over shuffles and merged into the list
// (one bitonic merge). Lists of different waves, of the row's history ids and of
// different chunks merge the same way. The finish (top-p, min-p, inverse-CDF draw in id
// order, fp64) runs in one wave over at most 64 candidates.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"

namespace arbor {

constexpr int kListSlots = kWaves;  // one list per wave

// Top-64 of two descending lists (lane i holds the i-th entry), descending.
__device__ __forceinline__ uint64_t list_merge(uint64_t a, uint64_t b) {
  const int lane = lane_id();
  const uint64_t rb = lane_reverse(b);
  uint64_t v = a > rb ? a : rb;  // bitonic, holds the 64 best of a and b
#pragma unroll
  for (int stride = kWave / 2; stride > 0; stride >>= 1) {
    const uint64_t w = lane_xor_n(v, stride);
    const bool lower = (lane & stride) == 0;
    const uint64_t mx = v > w ? v : w, mn = v > w ? w : v;
    v = lower ? mx : mn;
  }
  return v;
}

__device__ __forceinline__ int list_count(uint64_t v) { return __popcll(__ballot(v != 0ull)); }

// z of entry k-1 of a list with at least k entries
__device__ __forceinline__ float list_kth_z(uint64_t v, int k) { return composite_z(lane_get(v, k - 1)); }

// The list shifted down by one lane (lane i gets lane i-1; DPP wave_shr:1, no LDS).
__device__ __forceinline__ uint64_t list_shift_down(uint64_t v) { return lane_shift_down(v, (uint64_t)0); }

// Insert composite c (wave-uniform) into a descending list, dropping the 64th entry.
__device__ __forceinline__ uint64_t list_insert(uint64_t best, uint64_t c) {
  const int lane = lane_id();
  const int pos = __popcll(__ballot(best > c));
  const uint64_t down = list_shift_down(best);
  return lane < pos ? best : (lane == pos ? c : down);
}

// Insert the lanes' pending candidates (bit q of `pend`: slot q, z = zof(q), id = idof(q))
// into the wave's list one at a time, skipping those that no longer reach the k-th entry
// once the list holds k. `thr` tracks the k-th z. Wave-uniform control flow.
template <int NQ, typename ZOf, typename IdOf>
__device__ __forceinline__ void list_absorb(uint64_t& best, float& thr, int k, uint32_t pend, ZOf zof, IdOf idof) {
  uint64_t kth = list_count(best) >= k ? lane_get(best, k - 1) : 0ull;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    uint64_t bal = __ballot((pend >> q) & 1u);
    if (!bal) continue;
    const uint64_t cq = composite(zof(q) + 0.0f, idof(q));
    while (bal) {
      const int src = __ffsll((long long)bal) - 1;
      bal &= bal - 1;
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)cq, src);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(cq >> 32), src);
      const uint64_t c = ((uint64_t)hi << 32) | lo;
      if (c <= kth) continue;
      best = list_insert(best, c);
      if (kth != 0ull || list_count(best) >= k) {
        const uint32_t klo = __builtin_amdgcn_readlane((uint32_t)best, k - 1);
        const uint32_t khi = __builtin_amdgcn_readlane((uint32_t)(best >> 32), k - 1);
        kth = ((uint64_t)khi << 32) | klo;
      }
    }
  }
  if (kth != 0ull) thr = fmaxf(thr, composite_z(kth));
}

// fp64 finish of a row from its sorted candidate list (lane i = i-th best, n >= 1 entries):
// top-p, then min-p, then the first id (ascending) whose running mass exceeds u * E.
// One wave; writes out_ids[row] and, if asked, the kept probabilities. u is the row's
// uniform (loaded early by callers that can).
__device__ __forceinline__ void finish_list(const Args& a, int row, uint64_t best, int n, float u) {
  const int lane = lane_id();
  const bool in = lane < n;
  const double z0 = (double)composite_z(lane_get(best, 0));
  const double e = in ? exp((double)composite_z(best) - z0) : 0.0;
  const double cum = wave_scan_incl(e);
  int lp = n;
  if (a.top_p < 1.0f) {
    const double target = (double)a.top_p * lane_get(cum, n - 1);
    const uint64_t hit = __ballot(in && cum >= target);
    if (hit) lp = __ffsll((long long)hit);
  }
  int kept = lp;
  if (a.min_p > 0.0f) {
    const uint64_t low = __ballot(lane < lp && e < (double)a.min_p);
    if (low) kept = __ffsll((long long)low) - 1;
  }
  // all n entries ordered by id (32-bit keys: marker bit 31 | id << 6 | rank; ids < 2^20),
  // independent of the filters above so that the two chains overlap; a sorted lane holds
  // a kept entry iff its rank is below `kept`
  const int32_t id = composite_id(best);
  uint32_t key = in ? (0x80000000u | ((uint32_t)id << 6) | (uint32_t)lane) : 0u;
  key = wave_sort64_desc_u32(key);  // descending: lanes [0, n), largest id first
  const int r = (int)(key & 63u);
  const bool kk = key != 0u && r < kept;
  const double er = __shfl(e, r);
  const double w = kk ? er : 0.0;
  // running mass in ascending id order = suffix sums over the descending lanes
  const double tot_w = wave_sum(w);
  const double cid = tot_w - wave_scan_incl(w) + w;  // sum over lanes >= this one
  const double E = tot_w;
  const double target = (double)u * E;
  // the ascending-first kept entry with running mass > target: the largest such lane
  // (lanes descend by id); none (rounding at u -> 1): the largest kept id, the first kept lane
  const uint64_t over = __ballot(kk && cid > target);
  const int pick = over ? 63 - __builtin_clzll(over) : __ffsll((long long)__ballot(kk)) - 1;
  const int32_t pick_id = (int32_t)((lane_get(key, pick) >> 6) & 0xFFFFFu);
  if (lane == 0) {
    a.out_ids[row] = pick_id;
    ring_append(a, row, pick_id);
  }
  if (a.write_probs && kk) a.out_probs[(size_t)row * (size_t)a.V + ((key >> 6) & 0xFFFFFu)] = (float)(er / E);
}
__device__ __forceinline__ void finish_list(const Args& a, int row, uint64_t best, int n) {
  finish_list(a, row, best, n, a.uniforms[row]);
}

}  // namespace arbor
