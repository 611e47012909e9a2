// split_solver.hpp -- the exact general path (top-p without top-k, plain sampling, top-k
// above the streaming limit) when the batch is smaller than the chip: S workgroups per
// row, one chunk of ids each, meeting at per-row barriers between phases. Each phase reads
// only its own chunk of the row (z is kept in the workspace) plus what the row's other
// chunks published.
//
// An ordinary launch, without co-residency: each workgroup takes its (row, chunk) from a
// ticket counter when it starts, so the tickets handed out are always a prefix in start
// order. Every row but the one holding the next ticket then has all of its workgroups
// running, and those wait only for each other; the one partial row waits for workgroups
// that start as soon as other rows finish and free their slots. So every barrier fills
// whatever share of the chip the grid gets (at least S workgroup slots).
//
//  1. Every workgroup builds the row's history table in LDS, writes its chunk of z
//     (penalties applied to the chunk's history ids) and publishes the chunk's statistics.
//  2. A cut (top-k by count, then top-p by mass; two or three barriers each): the chunks
//     publish 4096-bin histograms over d = zmax - z (the bins of mass_solver.hpp); every
//     workgroup sums the row's S histograms and finds the bin holding the target, so all of
//     them pick the same bin; when that bin holds more than kFsColl entries, the same again
//     within it; then the chunks publish the entries of the selected bin or sub-bin and
//     every workgroup ranks all of them and finds the same cut. More
//     entries than kFsColl (heavy ties) send the row to the radix solver, which the row's
//     first workgroup runs alone.
//  3. The draw (one barrier): the chunks publish their kept fixed-point mass and last kept
//     id; the workgroup whose chunk holds the crossing of floor(u * E) in id order scans it.
// Masses are the fixed-point ones of mass_solver.hpp, so every sum is exact and the result
// does not depend on the split.
#pragma once

#include "mass_solver.hpp"

namespace arbor {

// What one chunk of a row publishes (workspace, one record per workgroup).
struct SplitChunk {
  uint32_t kmax, kmin, nf, flags;  // order-key range of finite z, finite count, flags
  unsigned long long kept_mass;     // fixed-point mass of the chunk's kept ids
  int32_t kept_last;                // largest kept id of the chunk (-1: none)
  int32_t ncoll;                    // entries of the selected sub-bin (may exceed kFsColl)
  // one histogram per level: a workgroup writes its level-1 histogram while others of the
  // row may still be reading its level-0 one (the next write to a level's histogram comes
  // two barriers later, after every reader has passed the barrier between); with the
  // totals of its 64 groups of 64 bins, so that a reader fetches the group totals and then
  // only the selected group's bins
  unsigned long long gcnt[2][kFsBins / 64];
  unsigned long long gmass[2][kFsBins / 64];
  uint32_t cnt[2][kFsBins];
  unsigned long long mass[2][kFsBins];
  unsigned long long coll_key[kFsColl];
  unsigned long long coll_m[kFsColl];
};

constexpr uint32_t kSplitSpinLimit = 1u << 26;  // seconds of waiting: a barrier that never fills is a bug

// Barrier of the workgroups of one row. *ctr counts arrivals over the whole call (zeroed
// before the launch, like the ticket counter and the row's failure word *fail); the n-th
// barrier of a row waits for n * S arrivals. Global writes made before it are visible to
// the row's other workgroups after it (agent-scope release before the arrival, acquire
// after the wait).
// A wait past `spin_limit` gives up: it sets the row's failure word (before any later
// arrival of this workgroup, so every workgroup that counts such an arrival sees it) and
// *timed_out. A workgroup that has timed out, or has seen the failure word, still arrives
// at every later barrier (so the counts stay whole) but waits at none and computes nothing
// more; the row's result is then ARBOR_ID_STALLED.
__device__ __forceinline__ void row_barrier(uint32_t* ctr, uint32_t* fail, uint32_t target, uint32_t spin_limit,
                                            int* timed_out) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    atomicAdd(ctr, 1u);
    if (!*timed_out) {
      uint32_t spins = 0u;
      while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        if (__hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
        __builtin_amdgcn_s_sleep(2);
        if (++spins >= spin_limit) {
          __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
      __threadfence();
      if (__hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) *timed_out = 1;
    }
  }
  __syncthreads();
}

// The row's id, written once every workgroup of the row is past its last barrier: a
// workgroup that timed out stores ARBOR_ID_STALLED unconditionally; the one that found the
// draw stores its id only if no ARBOR_ID_STALLED is there, so the sentinel wins whichever
// store comes first.
__device__ __forceinline__ void store_row_id(int32_t* out, int32_t id) {
  int32_t cur = __hip_atomic_load(out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (cur != ARBOR_ID_STALLED) {
    if (__hip_atomic_compare_exchange_strong(out, &cur, id, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      break;
  }
}

template <int DT>
__global__ void __launch_bounds__(kBlock) split_solver_kernel(Args a, SplitChunk* chunks, uint32_t* ctr,
                                                               uint32_t spin_limit) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* htab = reinterpret_cast<uint32_t*>(smem);
  FastShared& sh = *reinterpret_cast<FastShared*>(smem + ((sizeof(uint32_t) << a.hash_bits) + 15) / 16 * 16);
  __shared__ int s_timeout;
  __shared__ uint32_t s_ticket;
  constexpr int NW = kWaves;
  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  // (row, chunk) in start order: ctr[B] is the ticket counter, ctr[0..B) the row barriers,
  // ctr[B + 1 + row] the rows' failure words
  if (t == 0) s_ticket = atomicAdd(ctr + a.B, 1u);
  __syncthreads();
  const int ticket = (int)s_ticket;
  const int S = a.S, row = ticket / S, chunk = ticket % S;
  const int V = a.V;
  const int c0 = chunk * a.chunk_len, c1 = min(V, c0 + a.chunk_len), n = c1 - c0;
  float* z = a.zbuf + (size_t)row * (size_t)a.ldz;  // the row's buffer; this workgroup owns [c0, c1)
  const float* zc = z + c0;
  SplitChunk* mine = chunks + ticket;
  const SplitChunk* rowc = chunks + (size_t)row * (size_t)S;
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = a.mask ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const int P = 1 << a.hash_bits;
  float* prow = a.write_probs ? a.out_probs + (size_t)row * (size_t)V : nullptr;
  uint32_t passed = 0u;  // row barriers passed
  if (t == 0) s_timeout = 0;
  uint32_t* fail_w = ctr + a.B + 1 + row;
  bool skip = false;  // this workgroup has nothing more to compute (it still meets every barrier)
  auto sync_row = [&]() {
    row_barrier(ctr + row, fail_w, ++passed * (uint32_t)S, spin_limit, &s_timeout);
    if (s_timeout) skip = true;
  };

  // ---- 1. history table, the chunk's z, its statistics ----
  uint32_t flags = 0u;
  // The chunk's history ids as a bitmap (in the histograms' mass array, unused until the
  // first cut) when it fits, so that penalties and statistics come with the one pass over
  // the logits; longer chunks penalise z in place and read it back for the statistics.
  const bool fused = n <= 64 * kFsBins;
  uint32_t* hbits = fused && a.H > 0 ? reinterpret_cast<uint32_t*>(sh.mass) : nullptr;
  if (a.H > 0) {
    for (int i = t; i < P; i += kBlock) htab[i] = kEmptySlot;
    if (hbits)
      for (int i = t; i < (n + 31) / 32; i += kBlock) hbits[i] = 0u;
    __syncthreads();
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    for (int j = t; j < a.H; j += kBlock) {
      const int32_t id = h[j];
      if (id < 0) continue;
      if (id >= V) {
        flags |= kFlagBadHistory;
      } else {
        hist_insert(htab, (uint32_t)a.hash_bits, (uint32_t)id);
        if (hbits && id >= c0 && id < c1) atomicOr(&hbits[(id - c0) >> 5], 1u << ((id - c0) & 31));
      }
    }
  }
  {
    uint32_t kmax = 0u, kmin = 0xFFFFFFFFu, nf = 0u;
    if (fused) {
      __syncthreads();  // history table and bitmap complete
      bool invalid = false;
      fs_temper_stats<kBlock, DT>(a, xrow, mrow, hbits, htab, z, c0, c1, kmax, kmin, nf, invalid);
      if (invalid) flags |= kFlagInvalid;
    } else {
      fs_temper<kBlock, DT>(a, xrow, mrow, z, c0, c1);
      __syncthreads();
      if (a.H > 0) {
        for (int sl = t; sl < P; sl += kBlock) {
          const uint32_t e = htab[sl];
          if (e == kEmptySlot) continue;
          const int id = (int)(e >> 12);
          if (id >= c0 && id < c1) z[id] = penalize(z[id], (e & 4095u) + 1u, a.pen);
        }
      }
      __syncthreads();
      fs_visit<kBlock>(zc, n, [&](int, float v) {
        if (is_invalid(v)) flags |= kFlagInvalid;
        if (v != -INFINITY && !is_invalid(v)) {
          const uint32_t k = order_key(v);
          kmax = k > kmax ? k : kmax;
          kmin = k < kmin ? k : kmin;
          ++nf;
        }
      });
    }
    flags = block_reduce_max<kBlock, uint32_t>(flags, sh.red32);
    kmax = block_reduce_max<kBlock, uint32_t>(kmax, sh.red32);
    kmin = block_reduce_min<kBlock, uint32_t>(kmin, sh.red32);
    nf = block_reduce_sum<kBlock, uint32_t>(nf, sh.red32);
    if (t == 0) {
      mine->kmax = kmax;
      mine->kmin = kmin;
      mine->nf = nf;
      mine->flags = flags;
    }
  }
  sync_row();

  // ---- row statistics (the same in every workgroup of the row) ----
  uint32_t kmax = 0u, kmin = 0xFFFFFFFFu, nf = 0u, rflags = 0u;
  for (int c = 0; c < S; ++c) {
    kmax = max(kmax, rowc[c].kmax);
    kmin = min(kmin, rowc[c].kmin);
    nf += rowc[c].nf;
    rflags |= rowc[c].flags;
  }
  if (!skip && (rflags != 0u || nf == 0u)) {
    if (chunk == 0 && t == 0)
      store_row_id(a.out_ids + row, (rflags & kFlagBadHistory)
                                        ? ARBOR_ID_BAD_HISTORY
                                        : ((rflags & kFlagInvalid) ? ARBOR_ID_INVALID : ARBOR_ID_EMPTY));
    if (prow)
      for (int i = c0 + t; i < c1; i += kBlock) prow[i] = 0.0f;
    skip = true;
  }
  const float zmax = key_value(kmax);
  const float span = fminf(zmax - key_value(kmin), kFsSpan);
  const float scale = (float)kFsBins / fmaxf(span, 0x1p-20f);

  // ---- 2. one cut over the split row (two barriers, three when the level-0 bin is large) ----
  auto split_cut = [&](bool by_mass, bool need_mass, uint64_t target, double frac) -> FsCut {
    FsCut r{0ull, 0ull, 0ull, false};
    uint64_t above_w = 0, above_c = 0, above_m = 0;
    int b0 = 0, b1 = 0;
    bool all = false;     // the whole row is below the target: keep everything
    bool direct = false;  // the level-0 bin is collected whole (no level 1)
    uint64_t sel_cnt = 0;  // entries of the selected bin
    for (int level = 0; level < 2; ++level) {
      if (!skip && !all) {
        for (int i = t; i < kFsBins; i += kBlock) {
          sh.cnt[i] = 0u;
          sh.mass[i] = 0ull;
        }
        __syncthreads();
        fs_visit<kBlock>(zc, n, [&](int, float v) {
          if (v == -INFINITY) return;
          const float x = fs_x(v, zmax, scale);
          int d = fs_bin0(x);
          if (level == 1) {
            if (d != b0) return;
            d = fs_bin1(x, b0);
          }
          // a mass cut needs counts only at level 0 (to size the selected bin); a count cut
          // needs masses only for a top-p after it
          if (!by_mass || level == 0) atomicAdd(&sh.cnt[d], 1u);
          if (need_mass) atomicAdd(&sh.mass[d], (unsigned long long)mass_fixed(rel_exp(v, zmax)));
        });
        __syncthreads();
        for (int i = t; i < kFsBins; i += kBlock) {
          mine->cnt[level][i] = sh.cnt[i];
          mine->mass[level][i] = sh.mass[i];
        }
        // group totals (group g = bins [64g, 64g + 64)): wave w sums groups w, w + 16, ...
#pragma unroll
        for (int j = 0; j < kFsBins / kBlock; ++j) {
          const int bin = j * kBlock + t;
          const uint64_t gc = wave_sum((uint64_t)sh.cnt[bin]);
          const uint64_t gm = wave_sum((uint64_t)sh.mass[bin]);
          if (lane == 0) {
            mine->gcnt[level][bin >> 6] = gc;
            mine->gmass[level][bin >> 6] = gm;
          }
        }
      }
      sync_row();
      if (!skip && !all) {
        // The row's bin, found by every wave on its own (the same in each: exact integer
        // sums): the row's 64 group totals (lane g: group g), the group in which the
        // running weight from the top reaches the target, then that group's 64 bins
        // (lane l: bin 64g + l) and the bin in which it does, as fs_find_bin finds it
        // over all 4096 bins. Weights are counts (by_mass false) or masses.
        uint64_t gc = 0, gm = 0;
        for (int c = 0; c < S; ++c) {
          gc += rowc[c].gcnt[level][lane];
          gm += rowc[c].gmass[level][lane];
        }
        if (level == 0 && frac > 0.0) {
          const uint64_t m = wave_sum(gm);
          const double tg = ceil(frac * (double)m);
          target = tg < 1.0 ? 1ull : (uint64_t)tg;
          if (target > m) target = m;
        }
        const uint64_t tgt = target - above_w;
        const uint64_t gw = by_mass ? gm : gc;
        const uint64_t gin = wave_scan_incl(gw);
        const uint64_t ghit = __ballot(gin - gw < tgt && gin >= tgt);
        if (ghit == 0ull) {
          all = true;  // the whole level is below the target: keep everything
        } else {
          const int g = __ffsll((long long)ghit) - 1;
          const uint64_t gex_c = lane_get(wave_scan_incl(gc) - gc, g);  // groups above g
          const uint64_t gex_m = lane_get(wave_scan_incl(gm) - gm, g);
          const uint64_t gex_w = by_mass ? gex_m : gex_c;
          uint64_t bc = 0, bm = 0;
          for (int c = 0; c < S; ++c) {
            bc += rowc[c].cnt[level][g * 64 + lane];
            bm += rowc[c].mass[level][g * 64 + lane];
          }
          const uint64_t bw = by_mass ? bm : bc;
          const uint64_t bin = gex_w + wave_scan_incl(bw);
          // the group's bins sum to its total, which reaches the target: one bin does
          const int l = __ffsll((long long)__ballot(bin - bw < tgt && bin >= tgt)) - 1;
          above_w += lane_get(bin - bw, l);
          above_c += gex_c + lane_get(wave_scan_incl(bc) - bc, l);
          above_m += gex_m + lane_get(wave_scan_incl(bm) - bm, l);
          sel_cnt = lane_get(bc, l);
          if (level == 0)
            b0 = g * 64 + l;
          else
            b1 = g * 64 + l;
        }
      }
      // a level-0 bin small enough to collect whole needs no level 1: every workgroup of the
      // row summed the same counts, so all of them leave here or none
      if (level == 0 && !skip && !all && sel_cnt <= (uint64_t)kFsColl) {
        direct = true;
        break;
      }
    }
    // the chunk's entries of the selected sub-bin
    if (!skip && !all) {
      if (t == 0) sh.b32[1] = 0;
      __syncthreads();
      fs_visit<kBlock>(zc, n, [&](int i, float v) {
        if (v == -INFINITY) return;
        const float x = fs_x(v, zmax, scale);
        if (fs_bin0(x) != b0 || (!direct && fs_bin1(x, b0) != b1)) return;
        const int pos = atomicAdd(&sh.b32[1], 1);
        if (pos < kFsColl) {
          mine->coll_key[pos] = composite(v, c0 + i);
          mine->coll_m[pos] = mass_fixed(rel_exp(v, zmax));
        }
      });
      __syncthreads();
      if (t == 0) mine->ncoll = sh.b32[1];
    }
    sync_row();
    if (skip || all) return r;
    // every chunk's entries, in chunk order, ranked by counting
    int ntot = 0;
    for (int c = 0; c < S; ++c) {
      const int nc = rowc[c].ncoll;
      if (nc > kFsColl || ntot + nc > kFsColl) {
        r.tied = true;
        return r;
      }
      for (int j = t; j < nc; j += kBlock) {
        const unsigned long long m = rowc[c].coll_m[j];
        sh.coll_key[ntot + j] = rowc[c].coll_key[j];
        sh.coll_m[ntot + j] = m;
        sh.coll_w[ntot + j] = by_mass ? m : 1ull;
      }
      ntot += nc;
    }
    __syncthreads();
    if (t < ntot) {
      const uint64_t c = sh.coll_key[t];
      int rank = 0;
      for (int j = 0; j < ntot; ++j) rank += sh.coll_key[j] > c ? 1 : 0;
      sh.mass[2 * rank] = c;
      sh.mass[2 * rank + 1] = (unsigned long long)t;
    }
    __syncthreads();
    uint64_t w = 0, m = 0, c = 0;
    if (t < ntot) {
      const int idx = (int)sh.mass[2 * t + 1];
      c = sh.mass[2 * t];
      w = sh.coll_w[idx];
      m = sh.coll_m[idx];
    }
    uint64_t totw, totm;
    const uint64_t exw = fs_scan_excl<kBlock>(w, sh.red64, &totw);
    const uint64_t exm = fs_scan_excl<kBlock>(m, sh.red64, &totm);
    if (t == 0) sh.b32[2] = -1;
    __syncthreads();
    if (t < ntot && above_w + exw < target && above_w + exw + w >= target) {
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
  };

  // cuts: top-k (count), then top-p (mass of the top-k survivors). Whether a cut runs is
  // decided from the arguments and the row statistics, so every workgroup of the row
  // meets the same barriers.
  uint64_t cut = 0ull;
  bool tied = false;
  uint64_t kept_mass = 0ull;
  if (a.top_k > 0 && (uint32_t)a.top_k < nf) {
    const FsCut ck = split_cut(false, a.top_p < 1.0f, (uint64_t)a.top_k, 0.0);
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
      cp = split_cut(true, true, target, 0.0);
    } else {
      cp = split_cut(true, true, 0ull, (double)a.top_p);
    }
    tied = cp.tied;
    if (cp.cut > cut) cut = cp.cut;
  }
  if (tied && !skip) {  // more entries in the final sub-bin than are ranked directly
    if (chunk == 0) solve_row<kBlock, DT>(a, row, htab, *reinterpret_cast<SolverShared*>(sh.cnt));
    skip = true;
  }
  const bool use_min_p = a.min_p > 0.0f;

  // ---- 3. draw: the chunk's kept mass, by waves over contiguous id ranges ----
  const int seg = (((n + NW - 1) / NW) + 4 * kWave - 1) / (4 * kWave) * (4 * kWave);
  const int r0 = min(n, wave * seg), r1 = min(n, r0 + seg);
  auto kept = [&](int i, float v, uint64_t* w) -> bool {  // i relative to c0
    *w = 0ull;
    if (i >= r1 || v == -INFINITY || composite(v, c0 + i) < cut) return false;
    const float e = rel_exp(v, zmax);
    if (use_min_p && !(e >= a.min_p)) return false;
    *w = mass_fixed(e);
    return true;
  };
  const fs_f4* zq = reinterpret_cast<const fs_f4*>(zc);
  uint64_t ws = 0;
  if (!skip) {
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
          if (kept(i, v[u][c], &w)) wl = c0 + i;
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
    const uint64_t ec = wave_sum(wsl);
    const int32_t lc = wave_max(lane < NW ? sh.wlast[lane] : -1);
    if (t == 0) {
      mine->kept_mass = ec;
      mine->kept_last = lc;
    }
  }
  sync_row();
  if (skip) {
    if (s_timeout && t == 0) __hip_atomic_exchange(a.out_ids + row, ARBOR_ID_STALLED, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  uint64_t E = 0, before = 0;
  int32_t last = -1;
  for (int c = 0; c < S; ++c) {
    const uint64_t m = rowc[c].kept_mass;
    E += m;
    if (c < chunk) before += m;
    last = max(last, (int32_t)rowc[c].kept_last);
  }
  const double uE = (double)a.uniforms[row] * (double)E;
  uint64_t target;
  if (uE >= 0.0)
    target = uE >= 18446744073709549568.0 ? ~0ull : (uint64_t)uE;
  else
    target = uE < 0.0 ? 0ull : ~0ull;  // NaN: no crossing
  const uint64_t ec = mine->kept_mass;
  if (before <= target && before + ec > target) {
    // this chunk holds the crossing: the wave whose range holds it scans its range
    const uint64_t wsl = lane < NW ? sh.wsum[lane] : 0ull;
    const uint64_t wbefore = before + wave_sum(lane < wave ? wsl : 0ull);
    if (t == 0) sh.b32[3] = -1;
    __syncthreads();
    if (wbefore <= target && wbefore + ws > target) {
      uint64_t run = wbefore;
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
            const uint64_t acc = incl - lw;
            int pick = i + 3;
#pragma unroll
            for (int c = 3; c >= 0; --c)
              if (acc + w[0] + (c > 0 ? w[1] : 0) + (c > 1 ? w[2] : 0) + (c > 2 ? w[3] : 0) > target) pick = i + c;
            sh.b32[3] = c0 + pick;
          }
          break;
        }
        run = lane_get(incl, kWave - 1);
      }
    }
    __syncthreads();
    if (t == 0) store_row_id(a.out_ids + row, sh.b32[3] >= 0 ? sh.b32[3] : last);
  } else if (target >= E && last >= c0 && last < c1) {
    if (t == 0) store_row_id(a.out_ids + row, last);  // no crossing (u * E rounds to E, or NaN u): the last kept id
  }
  if (prow) {
    const double Ed = (double)E / (double)kMassScale;
    fs_visit<kBlock>(zc, n, [&](int i, float v) {
      float q = 0.0f;
      if (v != -INFINITY && composite(v, c0 + i) >= cut) {
        const float e = rel_exp(v, zmax);
        if (!use_min_p || e >= a.min_p) q = (float)((double)e / Ed);
      }
      prow[c0 + i] = q;
    });
  }
}

__global__ void zero_u32_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace arbor
