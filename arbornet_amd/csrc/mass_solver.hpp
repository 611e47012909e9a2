// mass_solver.hpp -- the exact general path, one workgroup of kBlock threads per row:
// top-p without top-k, plain sampling, top-k above the streaming limit.
//
// The row's z is materialised in the workspace (one read of the logits from HBM); every
// later pass reads it back from the caches. A cut (top-k by count, top-p by probability
// mass) is found with two levels of 4096-bin histograms over the distance below the row
// maximum, d = zmax - z: level 0 splits [0, span) into 4096 bins (span = min(zmax - zmin,
// 32); beyond 32 every fixed-point mass is zero), and when the bin that holds the target
// has more than kFsColl entries, level 1 splits it into 4096 more. Both bin functions are
// monotone in z (float rounding is monotone), so bins are contiguous ranges of the rank
// order; the entries of the final bin or sub-bin are collected and ranked by their 64-bit
// rank key. Masses are fixed point
// (exp(z - zmax) in units of 2^-40, summed in uint64), so every sum is exact and the cut
// and the draw are the same as those of the radix solver (row_solver.hpp), which remains
// the fallback for rows with more than kFsColl entries in one sub-bin (ties).
// The draw: per-wave sums of the kept mass over contiguous id ranges, then the wave whose
// range holds the crossing scans it in id order.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"
#include "row_solver.hpp"

namespace arbor {

constexpr int kFsBins = 4096;  // bins per histogram level
constexpr float kFsSpan = 32.0f;  // widest d = zmax - z histogrammed; masses beyond are zero
constexpr int kFsColl = 1024;  // entries of the final sub-bin ranked directly

struct FastShared {
  uint32_t cnt[kFsBins];
  unsigned long long mass[kFsBins];  // after a level: the collected entries, sorted
  uint64_t coll_key[kFsColl];
  uint64_t coll_w[kFsColl];
  uint64_t coll_m[kFsColl];
  uint64_t red64[kWaves];
  uint32_t red32[kWaves];
  uint64_t wsum[kWaves];
  int32_t wlast[kWaves];
  uint64_t b64[4];
  int32_t b32[4];
};
static_assert(sizeof(SolverShared) <= sizeof(uint32_t) * kFsBins, "radix-solver scratch fits the count bins");

// Integer block sum and exclusive scan whose cross-wave step is a wave reduction over
// the per-wave partials (lane w holds wave w's), so no thread keeps all partials live.
template <int BLOCK>
__device__ __forceinline__ uint64_t fs_sum(uint64_t v, uint64_t* scratch) {
  constexpr int NW = BLOCK / kWave;
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) scratch[threadIdx.x / kWave] = v;
  __syncthreads();
  const uint64_t r = wave_sum(lane_id() < NW ? scratch[lane_id()] : 0ull);
  __syncthreads();
  return r;
}

template <int BLOCK>
__device__ __forceinline__ uint64_t fs_scan_excl(uint64_t v, uint64_t* scratch, uint64_t* total) {
  constexpr int NW = BLOCK / kWave;
  const uint64_t incl = wave_scan_incl(v);
  const int w = threadIdx.x / kWave, lane = lane_id();
  __syncthreads();
  if (lane == kWave - 1) scratch[w] = incl;
  __syncthreads();
  const uint64_t s = lane < NW ? scratch[lane] : 0ull;
  const uint64_t base = wave_sum(lane < w ? s : 0ull);
  *total = wave_sum(s);
  __syncthreads();
  return base + incl - v;
}

struct FsCut {
  uint64_t cut;    // kept iff composite >= cut (0: keep everything)
  uint64_t count;  // entries kept
  uint64_t mass;   // fixed-point mass kept
  bool tied;       // more than kFsColl entries in the final sub-bin: no cut found
};

constexpr int kFsLoads = 4;  // 16-byte loads in flight per thread in a pass over z

typedef float fs_f4 __attribute__((ext_vector_type(4)));

// f(i, z[i]) for every i in [0, V): z is a 16-byte aligned row padded to a multiple of 4
// floats; each thread reads 4 consecutive entries per load, kFsLoads loads in flight.
template <int BLOCK, typename F>
__device__ __forceinline__ void fs_visit(const float* z, int V, F f) {
  const int nq = (V + 3) >> 2;
  const fs_f4* zq = reinterpret_cast<const fs_f4*>(z);
  for (int base = threadIdx.x; base < nq; base += BLOCK * kFsLoads) {
    fs_f4 v[kFsLoads];
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int q = base + u * BLOCK;
      v[u] = q < nq ? zq[q] : fs_f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int i0 = 4 * (base + u * BLOCK);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (i0 + c < V) f(i0 + c, v[u][c]);
    }
  }
}

// Tempered, masked logits z[i] = x[i] * (1/T) (or -inf where the mask clears i) for i in
// [c0, c1), c0 a multiple of 32: VEC-entry units, kFsLoads units in flight per thread.
// z is the row's padded buffer (16-byte aligned, room up to the next multiple of 64).
template <int BLOCK, int DT>
__device__ __forceinline__ void fs_temper(const Args& a, const void* xrow, const uint32_t* mrow, float* z, int c0,
                                          int c1) {
  constexpr int VEC = Elem<DT>::kVec;
  const bool aligned = a.aligned != 0;
  const int nu = (c1 - c0 + VEC - 1) / VEC;
  for (int base = threadIdx.x; base < nu; base += BLOCK * kFsLoads) {
    float x[kFsLoads][VEC];
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int q = base + u * BLOCK;
      if (q < nu) load_unit<DT>(xrow, c0 + q * VEC, c1, aligned, x[u]);
    }
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int q = base + u * BLOCK;
      if (q >= nu) continue;
      const int e0 = c0 + q * VEC;
      const uint32_t bits = mrow ? mrow[e0 >> 5] >> (e0 & 31) : 0xFFFFFFFFu;
#pragma unroll
      for (int c = 0; c < VEC; c += 4) {
        fs_f4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = x[u][c + j] * a.inv_t + 0.0f;
          o[j] = ((bits >> (c + j)) & 1u) ? v : -INFINITY;
        }
        if (e0 + c < c1) *reinterpret_cast<fs_f4*>(z + e0 + c) = o;
      }
    }
  }
}

// fs_temper with the penalties and the statistics in the same pass: ids whose bit
// (i - c0) is set in hbits are history ids (counts from the row's history table) and are
// penalised as they are written, with the same operations in the same order as a
// separate penalty pass over z. Returns, over the written z: the order-key range and the
// number of finite entries, and whether any entry is invalid (NaN or +inf).
template <int BLOCK, int DT>
__device__ __forceinline__ void fs_temper_stats(const Args& a, const void* xrow, const uint32_t* mrow,
                                                const uint32_t* hbits, const uint32_t* htab, float* z, int c0,
                                                int c1, uint32_t& kmax, uint32_t& kmin, uint32_t& nf, bool& invalid) {
  constexpr int VEC = Elem<DT>::kVec;
  static_assert(32 % VEC == 0, "a unit's history bits lie in one bitmap word");
  const bool aligned = a.aligned != 0;
  const int nu = (c1 - c0 + VEC - 1) / VEC;
  for (int base = threadIdx.x; base < nu; base += BLOCK * kFsLoads) {
    float x[kFsLoads][VEC];
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int q = base + u * BLOCK;
      if (q < nu) load_unit<DT>(xrow, c0 + q * VEC, c1, aligned, x[u]);
    }
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int q = base + u * BLOCK;
      if (q >= nu) continue;
      const int e0 = c0 + q * VEC;
      const uint32_t bits = mrow ? mrow[e0 >> 5] >> (e0 & 31) : 0xFFFFFFFFu;
      const uint32_t hb = hbits ? hbits[(e0 - c0) >> 5] >> ((e0 - c0) & 31) : 0u;
#pragma unroll
      for (int c = 0; c < VEC; c += 4) {
        fs_f4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v = x[u][c + j] * a.inv_t + 0.0f;
          v = ((bits >> (c + j)) & 1u) ? v : -INFINITY;
          if ((hb >> (c + j)) & 1u) v = penalize(v, hist_count(htab, (uint32_t)a.hash_bits, (uint32_t)(e0 + c + j)), a.pen);
          o[j] = v;
          if (e0 + c + j < c1) {
            const bool bad = is_invalid(v);
            invalid |= bad;
            if (v != -INFINITY && !bad) {
              const uint32_t k = order_key(v);
              kmax = k > kmax ? k : kmax;
              kmin = k < kmin ? k : kmin;
              ++nf;
            }
          }
        }
        if (e0 + c < c1) *reinterpret_cast<fs_f4*>(z + e0 + c) = o;
      }
    }
  }
}

// Level-0 bin of d = zmax - v (scale = kFsBins / span), and the level-1 sub-bin of an
// entry of level-0 bin b0. Non-decreasing in d, i.e. bins ascend as the rank descends.
__device__ __forceinline__ float fs_x(float v, float zmax, float scale) { return (zmax - v) * scale; }
// Bin indices are clamped to [0, kFsBins) whatever x is (NaN reads as 0).
__device__ __forceinline__ int fs_bin0(float x) {
  return x >= (float)(kFsBins - 1) ? kFsBins - 1 : (int)fmaxf(x, 0.0f);
}
__device__ __forceinline__ int fs_bin1(float x, int b0) {
  const float y = (x - (float)b0) * (float)kFsBins;
  return y >= (float)(kFsBins - 1) ? kFsBins - 1 : (int)fmaxf(y, 0.0f);
}

// The bin (in ascending bin order, i.e. descending rank) at which the running weight of bins, from the top,
// reaches `target`; every thread gets the bin and the weight of the bins above it.
// w(b) = cnt[b] (by_mass false) or mass[b]. Returns -1 if the total is below target.
template <int BLOCK>
__device__ int fs_find_bin(FastShared& sh, bool by_mass, uint64_t target, uint64_t* above) {
  constexpr int PER = kFsBins / BLOCK;
  static_assert(kFsBins % BLOCK == 0, "bins split evenly over the threads");
  const int t = threadIdx.x;
  uint64_t w[PER];
  uint64_t loc = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int b = t * PER + j;
    w[j] = by_mass ? (uint64_t)sh.mass[b] : (uint64_t)sh.cnt[b];
    loc += w[j];
  }
  uint64_t tot;
  const uint64_t ex = fs_scan_excl<BLOCK>(loc, sh.red64, &tot);
  if (t == 0) sh.b32[0] = -1;
  __syncthreads();
  if (ex < target && ex + loc >= target) {
    uint64_t run = ex;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (run + w[j] >= target) {
        sh.b32[0] = t * PER + j;
        sh.b64[0] = run;
        break;
      }
      run += w[j];
    }
  }
  __syncthreads();
  const int b = sh.b32[0];
  *above = sh.b64[0];
  __syncthreads();
  return b;
}

// Cut of the row z[0, V) at `target` (count, or fixed-point mass; if frac > 0 the target
// is ceil(frac * total mass)): the first entry in rank order at which the running weight
// reaches the target. Counts and masses of the kept set are returned for both modes.
template <int BLOCK>
__device__ FsCut fs_cut(const float* z, int V, float zmax, float scale, bool by_mass, uint64_t target, double frac,
                        FastShared& sh) {
  const int t = threadIdx.x;
  FsCut r{0ull, 0ull, 0ull, false};
  uint64_t above_w = 0, above_c = 0, above_m = 0;
  int b0 = 0, b1 = 0;    // selected bins
  bool direct = false;  // the level-0 bin is collected whole (no level 1)
  for (int level = 0; level < 2; ++level) {
    for (int i = t; i < kFsBins; i += BLOCK) {
      sh.cnt[i] = 0u;
      sh.mass[i] = 0ull;
    }
    __syncthreads();
    fs_visit<BLOCK>(z, V, [&](int, float v) {
      if (v == -INFINITY) return;
      const float x = fs_x(v, zmax, scale);
      int d = fs_bin0(x);
      if (level == 1) {
        if (d != b0) return;
        d = fs_bin1(x, b0);
      }
      atomicAdd(&sh.cnt[d], 1u);
      atomicAdd(&sh.mass[d], (unsigned long long)mass_fixed(rel_exp(v, zmax)));
    });
    __syncthreads();
    if (level == 0 && frac > 0.0) {
      uint64_t m = 0;
      for (int b = t; b < kFsBins; b += BLOCK) m += sh.mass[b];
      m = fs_sum<BLOCK>(m, sh.red64);
      const double tg = ceil(frac * (double)m);
      target = tg < 1.0 ? 1ull : (uint64_t)tg;
      if (target > m) target = m;
    }
    uint64_t above;
    const int b = fs_find_bin<BLOCK>(sh, by_mass, target - above_w, &above);
    if (b < 0) return r;  // the whole row is below the target: keep everything
    // counts and masses of the bins ranked above the selected one
    uint64_t ac = 0, am = 0;
    for (int j = t; j < kFsBins; j += BLOCK)
      if (j < b) {
        ac += sh.cnt[j];
        am += sh.mass[j];
      }
    ac = fs_sum<BLOCK>(ac, sh.red64);
    am = fs_sum<BLOCK>(am, sh.red64);
    above_w += above;
    above_c += ac;
    above_m += am;
    if (level == 0) {
      b0 = b;
      // a bin small enough to collect whole needs no level 1
      const bool small = sh.cnt[b0] <= (uint32_t)kFsColl;
      __syncthreads();  // every thread has read the count before level 1 clears the bins
      if (small) {
        direct = true;
        break;
      }
    } else {
      b1 = b;
    }
  }
  // entries of the selected bin or sub-bin: collect, rank by counting, run the target down
  if (t == 0) sh.b32[1] = 0;
  __syncthreads();
  fs_visit<BLOCK>(z, V, [&](int i, float v) {
    if (v == -INFINITY) return;
    const float x = fs_x(v, zmax, scale);
    if (fs_bin0(x) != b0 || (!direct && fs_bin1(x, b0) != b1)) return;
    const int pos = atomicAdd(&sh.b32[1], 1);
    if (pos < kFsColl) {
      const uint64_t m = mass_fixed(rel_exp(v, zmax));
      sh.coll_key[pos] = composite(v, i);
      sh.coll_m[pos] = m;
      sh.coll_w[pos] = by_mass ? m : 1ull;
    }
  });
  __syncthreads();
  const int n = sh.b32[1];
  if (n > kFsColl) {  // more entries in one sub-bin than the collector holds
    r.tied = true;
    return r;
  }
  // sorted order into the (free) bins: mass[2r] = key, mass[2r + 1] = index
  if (t < n) {
    const uint64_t c = sh.coll_key[t];
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += sh.coll_key[j] > c ? 1 : 0;
    sh.mass[2 * rank] = c;
    sh.mass[2 * rank + 1] = (unsigned long long)t;
  }
  __syncthreads();
  uint64_t w = 0, m = 0;
  uint64_t c = 0;
  if (t < n) {
    const int idx = (int)sh.mass[2 * t + 1];
    c = sh.mass[2 * t];
    w = sh.coll_w[idx];
    m = sh.coll_m[idx];
  }
  uint64_t totw, totm;
  const uint64_t exw = fs_scan_excl<BLOCK>(w, sh.red64, &totw);
  const uint64_t exm = fs_scan_excl<BLOCK>(m, sh.red64, &totm);
  if (t == 0) sh.b32[2] = -1;
  __syncthreads();
  if (t < n && above_w + exw < target && above_w + exw + w >= target) {
    sh.b32[2] = t;
    sh.b64[1] = c;
    sh.b64[2] = above_c + (uint64_t)t + 1;
    sh.b64[3] = above_m + exm + m;
  }
  __syncthreads();
  if (sh.b32[2] >= 0) {
    r.cut = sh.b64[1];
    r.count = sh.b64[2];
    r.mass = sh.b64[3];
  }
  __syncthreads();
  return r;
}

// The full contract for one row by one workgroup of BLOCK threads. htab has
// 1 << a.hash_bits slots of LDS.
template <int BLOCK, int DT>
__device__ void solve_row_fast(const Args& a, int row, uint32_t* htab, FastShared& sh) {
  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  constexpr int NW = BLOCK / kWave;
  const int V = a.V;
  float* z = a.zbuf + (size_t)row * (size_t)a.ldz;
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = a.mask ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const int P = 1 << a.hash_bits;

  // 1. history table of the whole row, and its ids as a bitmap (in the histograms' mass
  // array, unused until the first cut) when the row fits in it. fp32 rows only: with bf16
  // units (8 entries) the fused pass spills in this kernel.
  uint32_t flags = 0;
  const bool fused = DT == ARBOR_DTYPE_F32 && V <= 64 * kFsBins;
  uint32_t* hbits = fused && a.H > 0 ? reinterpret_cast<uint32_t*>(sh.mass) : nullptr;
  if (a.H > 0) {
    for (int i = t; i < P; i += BLOCK) htab[i] = kEmptySlot;
    if (hbits)
      for (int i = t; i < (V + 31) / 32; i += BLOCK) hbits[i] = 0u;
    __syncthreads();
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    for (int j = t; j < a.H; j += BLOCK) {
      const int32_t id = h[j];
      if (id < 0) continue;
      if (id >= V) {
        flags |= kFlagBadHistory;
      } else {
        hist_insert(htab, (uint32_t)a.hash_bits, (uint32_t)id);
        if (hbits) atomicOr(&hbits[id >> 5], 1u << (id & 31));
      }
    }
  }
  uint32_t kmax = 0, kmin = 0xFFFFFFFFu, nf = 0;
  if (fused) {
    // 2-4. tempered, masked, penalised logits and the row statistics in one pass
    __syncthreads();  // history table and bitmap complete
    bool invalid = false;
    fs_temper_stats<BLOCK, DT>(a, xrow, mrow, hbits, htab, z, 0, V, kmax, kmin, nf, invalid);
    if (invalid) flags |= kFlagInvalid;
  } else {
    // 2. tempered, masked logits
    fs_temper<BLOCK, DT>(a, xrow, mrow, z, 0, V);
    __syncthreads();
    // 3. penalties, one writer per distinct history id
    if (a.H > 0) {
      for (int s = t; s < P; s += BLOCK) {
        const uint32_t e = htab[s];
        if (e == kEmptySlot) continue;
        const uint32_t id = e >> 12;
        z[id] = penalize(z[id], (e & 4095u) + 1u, a.pen);
      }
    }
    __syncthreads();
    // 4. row statistics
    fs_visit<BLOCK>(z, V, [&](int, float v) {
      if (is_invalid(v)) flags |= kFlagInvalid;
      if (v != -INFINITY && !is_invalid(v)) {
        const uint32_t k = order_key(v);
        kmax = k > kmax ? k : kmax;
        kmin = k < kmin ? k : kmin;
        ++nf;
      }
    });
  }
  flags = block_reduce_max<BLOCK, uint32_t>(flags & kFlagBadHistory ? 2u : (flags & kFlagInvalid ? 1u : 0u),
                                            sh.red32);
  kmax = block_reduce_max<BLOCK, uint32_t>(kmax, sh.red32);
  kmin = block_reduce_min<BLOCK, uint32_t>(kmin, sh.red32);
  nf = block_reduce_sum<BLOCK, uint32_t>(nf, sh.red32);
  float* prow = a.write_probs ? a.out_probs + (size_t)row * (size_t)V : nullptr;
  if (flags != 0 || nf == 0) {
    if (t == 0) a.out_ids[row] = flags == 2u ? ARBOR_ID_BAD_HISTORY : (flags == 1u ? ARBOR_ID_INVALID : ARBOR_ID_EMPTY);
    if (prow)
      for (int i = t; i < V; i += BLOCK) prow[i] = 0.0f;
    return;
  }
  const float zmax = key_value(kmax);
  const float span = fminf(zmax - key_value(kmin), kFsSpan);  // NaN-free: both finite
  const float scale = (float)kFsBins / fmaxf(span, 0x1p-20f);

  // 5. cuts: top-k (count), then top-p (mass of the top-k survivors)
  uint64_t cut = 0ull;
  bool tied = false;
  uint64_t kept_mass = 0ull;
  if (a.top_k > 0 && (uint32_t)a.top_k < nf) {
    const FsCut ck = fs_cut<BLOCK>(z, V, zmax, scale, false, (uint64_t)a.top_k, 0.0, sh);
    tied = ck.tied;
    cut = ck.cut;
    kept_mass = ck.mass;
  }
  if (!tied && a.top_p < 1.0f) {
    FsCut cp;
    if (cut != 0ull) {
      const double tg = ceil((double)a.top_p * (double)kept_mass);
      uint64_t target = tg < 1.0 ? 1ull : (uint64_t)tg;
      if (target > kept_mass) target = kept_mass;
      cp = fs_cut<BLOCK>(z, V, zmax, scale, true, target, 0.0, sh);
    } else {
      cp = fs_cut<BLOCK>(z, V, zmax, scale, true, 0ull, (double)a.top_p, sh);
    }
    tied = cp.tied;
    if (cp.cut > cut) cut = cp.cut;
  }
  if (tied) {  // rare: more than kFsColl entries in one sub-bin
    solve_row<BLOCK, DT>(a, row, htab, *reinterpret_cast<SolverShared*>(sh.cnt));
    return;
  }
  const bool use_min_p = a.min_p > 0.0f;

  // 6. draw: kept mass of each wave's contiguous id range, then the wave holding the
  // crossing of floor(u * E) scans its range in id order
  const int seg = (((V + NW - 1) / NW) + 4 * kWave - 1) / (4 * kWave) * (4 * kWave);
  const int r0 = min(V, wave * seg), r1 = min(V, r0 + seg);
  // kept entry i of z (value v): *w its fixed-point mass
  auto kept = [&](int i, float v, uint64_t* w) -> bool {
    *w = 0ull;
    if (i >= r1 || v == -INFINITY || composite(v, i) < cut) return false;
    const float e = rel_exp(v, zmax);
    if (use_min_p && !(e >= a.min_p)) return false;
    *w = mass_fixed(e);
    return true;
  };
  const fs_f4* zq = reinterpret_cast<const fs_f4*>(z);
  uint64_t ws = 0;
  int32_t wl = -1;
  for (int i0 = r0 + 4 * lane; i0 < r1; i0 += 4 * kWave * kFsLoads) {
    fs_f4 v[kFsLoads];
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u) {
      const int i = i0 + 4 * kWave * u;
      v[u] = i < r1 ? zq[i >> 2] : fs_f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
#pragma unroll
    for (int u = 0; u < kFsLoads; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = i0 + 4 * kWave * u + c;
        uint64_t w;
        if (kept(i, v[u][c], &w)) wl = i;
        ws += w;
      }
  }
  ws = wave_sum(ws);
  wl = wave_max(wl);
  if (lane == 0) {
    sh.wsum[wave] = ws;
    sh.wlast[wave] = wl;
  }
  __syncthreads();
  const uint64_t wsl = lane < NW ? sh.wsum[lane] : 0ull;
  const uint64_t E = wave_sum(wsl);
  const uint64_t before = wave_sum(lane < wave ? wsl : 0ull);
  const int32_t last = wave_max(lane < NW ? sh.wlast[lane] : -1);
  const double uE = (double)a.uniforms[row] * (double)E;
  uint64_t target;
  if (uE >= 0.0)
    target = uE >= 18446744073709549568.0 ? ~0ull : (uint64_t)uE;
  else
    target = uE < 0.0 ? 0ull : ~0ull;  // NaN: no crossing
  if (t == 0) sh.b32[3] = -1;
  __syncthreads();
  if (before <= target && before + ws > target) {
    uint64_t run = before;
    for (int i0 = r0; i0 < r1; i0 += 4 * kWave) {
      const int i = i0 + 4 * lane;
      const fs_f4 v = i < r1 ? zq[i >> 2] : fs_f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      uint64_t w[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) kept(i + c, v[c], &w[c]);
      const uint64_t lw = w[0] + w[1] + w[2] + w[3];
      const uint64_t incl = run + wave_scan_incl(lw);
      const uint64_t hit = __ballot(incl > target);
      if (hit) {
        if (lane == __ffsll((long long)hit) - 1) {
          uint64_t acc = incl - lw;
          int pick = i + 3;
#pragma unroll
          for (int c = 3; c >= 0; --c)
            if (acc + w[0] + (c > 0 ? w[1] : 0) + (c > 1 ? w[2] : 0) + (c > 2 ? w[3] : 0) > target) pick = i + c;
          sh.b32[3] = pick;
        }
        break;
      }
      run = lane_get(incl, kWave - 1);
    }
  }
  __syncthreads();
  if (t == 0) a.out_ids[row] = sh.b32[3] >= 0 ? sh.b32[3] : last;
  if (prow) {
    const double Ed = (double)E / (double)kMassScale;
    fs_visit<BLOCK>(z, V, [&](int i, float v) {
      float q = 0.0f;
      if (v != -INFINITY && composite(v, i) >= cut) {
        const float e = rel_exp(v, zmax);
        if (!use_min_p || e >= a.min_p) q = (float)((double)e / Ed);
      }
      prow[i] = q;
    });
  }
}

}  // namespace arbor
