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

constexpr int kListSlots = kWaves + 1;  // the waves' lists plus the history list

// Top-64 of two descending lists (lane i holds the i-th entry), descending.
__device__ __forceinline__ uint64_t list_merge(uint64_t a, uint64_t b) {
  const int lane = lane_id();
  const uint64_t rb = __shfl(b, kWave - 1 - lane);
  uint64_t v = a > rb ? a : rb;  // bitonic, holds the 64 best of a and b
#pragma unroll
  for (int stride = kWave / 2; stride > 0; stride >>= 1) {
    const uint64_t w = __shfl_xor(v, stride);
    const bool lower = (lane & stride) == 0;
    const uint64_t mx = v > w ? v : w, mn = v > w ? w : v;
    v = lower ? mx : mn;
  }
  return v;
}

__device__ __forceinline__ int list_count(uint64_t v) { return __popcll(__ballot(v != 0ull)); }

// z of entry k-1 of a list with at least k entries
__device__ __forceinline__ float list_kth_z(uint64_t v, int k) { return composite_z(__shfl(v, k - 1)); }

// Collect the lanes' pending candidates (bit q of `pend`: slot q, z = zof(q), id = idof(q))
// into the wave's list, 64 at a time; once the list holds k entries `thr` rises to its
// k-th z and pending slots below it are dropped. Wave-uniform control flow. scratch: 64
// LDS entries private to this wave.
template <int NQ, typename ZOf, typename IdOf>
__device__ __forceinline__ void list_absorb(uint64_t& best, float& thr, int k, uint32_t pend, ZOf zof, IdOf idof,
                                            uint64_t* scratch) {
  const int lane = lane_id();
  while (__ballot(pend != 0u)) {
    int base = 0;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const bool tk = (pend >> q) & 1u;
      const uint64_t bal = __ballot(tk);
      if (bal) {
        const int pos = base + lanes_below(bal);
        if (tk && pos < kWave) {
          scratch[pos] = composite(zof(q) + 0.0f, idof(q));
          pend &= ~(1u << q);
        }
        base += __popcll(bal);
      }
    }
    wave_lds_sync();
    const int n = base < kWave ? base : kWave;
    uint64_t v = lane < n ? scratch[lane] : 0ull;
    wave_lds_sync();
    v = wave_sort64_desc(v);
    best = list_merge(best, v);
    if (list_count(best) >= k) thr = fmaxf(thr, list_kth_z(best, k));
    if (pend) {
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        if (((pend >> q) & 1u) && !(zof(q) >= thr)) pend &= ~(1u << q);
    }
  }
}

// fp64 finish of a row from its sorted candidate list (lane i = i-th best, n >= 1 entries):
// top-p, then min-p, then the first id (ascending) whose running mass exceeds u * E.
// One wave; writes out_ids[row] and, if asked, the kept probabilities.
__device__ void finish_list(const Args& a, int row, uint64_t best, int n) {
  const int lane = lane_id();
  const bool in = lane < n;
  const double z0 = (double)composite_z(__shfl(best, 0));
  const double e = in ? exp((double)composite_z(best) - z0) : 0.0;
  const double cum = wave_scan_incl(e);
  int lp = n;
  if (a.top_p < 1.0f) {
    const double target = (double)a.top_p * __shfl(cum, n - 1);
    const uint64_t hit = __ballot(in && cum >= target);
    if (hit) lp = __ffsll((long long)hit);
  }
  int kept = lp;
  if (a.min_p > 0.0f) {
    const uint64_t low = __ballot(lane < lp && e < (double)a.min_p);
    if (low) kept = __ffsll((long long)low) - 1;
  }
  // kept ranks [0, kept): order them by id, running mass in id order
  const int32_t id = composite_id(best);
  uint64_t key = lane < kept ? (((uint64_t)(uint32_t)id << 32) | (uint32_t)lane) : ~0ull;
  key = ~wave_sort64_desc(~key);  // ascending
  const int r = (int)(uint32_t)key;
  const double er = __shfl(e, lane < kept ? r : 0);
  const double w = lane < kept ? er : 0.0;
  const double cid = wave_scan_incl(w);
  const double E = __shfl(cid, kept - 1);
  const double target = (double)a.uniforms[row] * E;
  const uint64_t over = __ballot(lane < kept && cid > target);
  const int pick = over ? __ffsll((long long)over) - 1 : kept - 1;
  const int32_t pick_id = (int32_t)(__shfl(key, pick) >> 32);
  if (lane == 0) a.out_ids[row] = pick_id;
  if (a.write_probs && lane < kept) a.out_probs[(size_t)row * (size_t)a.V + (key >> 32)] = (float)(er / E);
}

}  // namespace arbor
