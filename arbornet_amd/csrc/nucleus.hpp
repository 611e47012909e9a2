// nucleus.hpp -- top-p without top-k (with or without min-p beside it) and sampling with
// no filter, in two passes over the logits with nothing written back: one 1024-thread
// workgroup per row, or, when the batch is smaller than the chip, S workgroups per row,
// each owning a chunk of ids, meeting at three per-row barriers.
//
//  1. Pass 1 streams the chunk from HBM once. Every final z (tempered, masked, penalised)
//     goes into an LDS histogram of 8192 bins of width 1/64 over [ref - 32, ref + 96);
//     ref is the largest final z of the row's first 512 (fp32) or 1024 (bf16) ids, which
//     every workgroup of the row computes alike. A bin word holds the count and the sum of
//     the entries' positions inside the bin (1/256 steps), so that
//     e^(c - ref) * (count + offsets / 64 + count / 98304) estimates the bin's mass to
//     ~1e-6 (c the bin centre; the last term is the mean second-order term). The chunk's
//     maximum comes with the pass. The estimates are summed per group of 64 bins; the
//     group, then the bin, where the running mass from the top reaches top_p of the total
//     are found (across the row's chunks: the group sums are exchanged first, then the 64
//     bins of the chosen group), and the bin of the min-p edge zmax + ln(min_p); b is the
//     higher (stricter) of the two.
//  2. Pass 2 reads the chunk again (from the caches: the 256 MB MALL holds it) and computes
//     each finite entry's mass e = exp(z - zmax) (fp32 exp2 with the rounding of the
//     argument folded back, accumulated in fp64 in a fixed order): all add to the total E;
//     entries in bins above b + 1 are kept whatever the exact cut and are summed per batch
//     of ids (one wave owns a batch); entries in bins b - 1 .. b + 1 are collected.
//  3. The collected entries of the whole row (exchanged between the row's chunks) are
//     sorted by rank key (counting sort into 1024 sub-bins, then in-place insertion sorts)
//     and the exact top-p cut is the first entry at which the running mass from the top
//     reaches top_p * E; min-p is then tested entry by entry. An estimate one bin off
//     still lands in the collected range; anything else (more entries than the collection
//     holds, heavy ties, a cut outside the range, an entry beyond the grid) sends the row
//     to the exact radix solver (row_solver.hpp).
//  4. The draw: the chunk whose running kept mass (in id order, across chunks) passes
//     u * E_kept adds its kept collected entries to their batches' sums, finds the batch
//     and rescans it in id order.
// Every sum is taken in a fixed order, so results do not depend on timing; the fp64
// estimates of pass 1 only choose which bins to collect.
//
// Barriers use tagged 64-bit words (call tag << 32 | count): the first arrival of a call
// replaces a stale word, so the workspace needs no clearing launch.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"
#include "row_solver.hpp"
#include "split_solver.hpp"

namespace arbor {

constexpr int kNuWaves = 16;
constexpr int kNuBlock = kNuWaves * kWave;        // 1024 threads
constexpr int kNuBins = 8192;                     // pass-1 grid
constexpr int kNuGroups = kNuBins / kWave;        // 128 groups of 64 bins
constexpr float kNuBelow = 32.0f;                 // the grid spans [ref - kNuBelow, ref + kNuAbove)
constexpr float kNuAbove = 96.0f;
constexpr float kNuScale = 64.0f;                 // bins per unit of z
constexpr int kNuColl = 4096;                     // collected entries of a row
constexpr int kNuCollChunk = 2048;                // collected entries one chunk may publish
constexpr int kNuSub = 1024;                      // sub-bins of the collected range (counting sort)
constexpr int kNuSubMax = 32;                     // entries a sub-bin sorts in place
constexpr int kNuBatchIds = 512;                  // ids per batch: 8 per lane (two fp32 units, one bf16 unit)
constexpr int kNuMaxChunk = 262144;               // ids per chunk (the history bitmap's reach)
constexpr uint32_t kNuFlagFallback = 8u;          // the row goes to the exact radix solver
constexpr uint32_t kNuSpinLimit = 1u << 26;       // seconds of waiting: a barrier that never fills is a bug
static_assert(kNuBins == 8 * kNuBlock, "eight bins per thread");
static_assert(kNuSub == kNuBlock, "one sub-bin per thread");
static_assert(kNuColl * (8 + 4 + 2) + kNuSub * 8 <= 8 * kNuBins, "the sort fits the histogram's LDS");
static_assert(sizeof(SolverShared) <= 8 * kNuBins, "the radix solver's scratch fits the histogram");

// What one chunk of a split row publishes (workspace, one record per workgroup).
struct NuRec {
  uint32_t kmax, flags;
  int32_t last, ncoll;
  double E, above;
  int32_t gsel, pad;
  double gsum[kNuGroups];   // estimated mass of each group of 64 bins (relative to ref)
  uint64_t gbins[kWave];    // the bin words of the selected group
  uint64_t ckey[kNuCollChunk];
  float cm[kNuCollChunk];
};

// Dynamic LDS of nucleus_kernel: histogram (then the collection and its sort) | group
// sums | batch sums (fp64, then fixed-point additions) | history bitmap | history table.
struct NuLayout {
  int gsum_off, seg_off, segx_off, bitmap_off, htab_off, bytes;
  __host__ __device__ static NuLayout make(int n_batches, int bitmap_words, int hash_slots) {
    NuLayout l;
    l.gsum_off = 8 * kNuBins;
    l.seg_off = l.gsum_off + 8 * kNuGroups;
    l.segx_off = l.seg_off + 8 * n_batches;
    l.bitmap_off = l.segx_off + 8 * n_batches;
    l.htab_off = l.bitmap_off + 4 * ((bitmap_words + 3) & ~3);
    l.bytes = l.htab_off + 4 * hash_slots;
    return l;
  }
};

// ---- tagged per-call counters (tag << 32 | count) ----
// The row's first workgroup stamps the row's words with the call's tag (count 0) when it
// starts; the others wait for the stamp before their first arrival, so no arrival of this
// call can be overwritten, and a word left over from an earlier call (or never written)
// reads as count 0.
__device__ __forceinline__ uint32_t tagged_count(const uint64_t* w, uint32_t tag) {
  const uint64_t v = __hip_atomic_load(const_cast<uint64_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (uint32_t)(v >> 32) == tag ? (uint32_t)v : 0u;
}
__device__ __forceinline__ bool tagged_is(const uint64_t* w, uint32_t tag) {
  const uint64_t v = __hip_atomic_load(const_cast<uint64_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (uint32_t)(v >> 32) == tag;
}

// Data a chunk publishes for its row goes through agent-coherent accesses (atomic loads and
// stores at agent scope bypass the XCDs' private L2s), so the barriers need no L2
// write-back or invalidation: an arrival waits only until this wave's stores completed.
template <typename T>
__device__ __forceinline__ void pub_store(T* p, T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit words");
  if constexpr (sizeof(T) == 4) {
    uint32_t b;
    __builtin_memcpy(&b, &v, 4);
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    uint64_t b;
    __builtin_memcpy(&b, &v, 8);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
template <typename T>
__device__ __forceinline__ T pub_load(const T* p) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit words");
  T v;
  if constexpr (sizeof(T) == 4) {
    const uint32_t b = __hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<T*>(p)), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_memcpy(&v, &b, 4);
  } else {
    const uint64_t b = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<T*>(p)), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_memcpy(&v, &b, 8);
  }
  return v;
}
// every memory operation this wave issued has completed
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Barrier of the workgroups of one row (see split_solver.hpp's row_barrier for the
// ordering argument): the n-th waits for n * S arrivals of this call, each one atomic add.
// A wait past the spin limit sets the row's failure word; a workgroup that gave up, or saw
// the word, still arrives everywhere but waits nowhere, and the row's result is
// ARBOR_ID_STALLED.
__device__ __forceinline__ void nu_barrier(uint64_t* ctr, uint64_t* fail, uint32_t tag, uint32_t target,
                                           uint32_t spin_limit, int* timed_out) {
  wait_all_memory();  // this wave's published stores are done (each wave before the block barrier)
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t spins = 0u;
    // the row's stamp (set by its first workgroup at its start) before the first arrival
    while (!*timed_out && !tagged_is(ctr, tag)) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins >= spin_limit) *timed_out = 1;
    }
    if (*timed_out) {
      __hip_atomic_store(fail, ((uint64_t)tag << 32) | 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __hip_atomic_fetch_add(ctr, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      while (tagged_count(ctr, tag) < target) {
        if (tagged_count(fail, tag) != 0u) break;
        __builtin_amdgcn_s_sleep(2);
        if (++spins >= spin_limit) {
          __hip_atomic_store(fail, ((uint64_t)tag << 32) | 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
      if (tagged_count(fail, tag) != 0u) *timed_out = 1;
    }
  }
  __syncthreads();
}

// exp(z - m) for z <= m, to ~1 ulp: the difference is taken exactly (TwoSum), its product
// with log2(e) keeps its rounding error, and the hardware exp2 result is corrected by it.
__device__ __forceinline__ float nu_exp(float z, float m) {
  constexpr float L = 1.44269502f;        // log2(e) rounded to fp32
  constexpr float Llo = 1.925963033e-8f;  // log2(e) - L
  const float d = z - m;
  const float bb = d - z;
  const float err = (z - (d - bb)) + (-m - bb);  // d + err == z - m exactly
  const float t = d * L;
  const float terr = __builtin_fmaf(d, L, -t) + (d * Llo + err * L);
  const float p = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(p * terr, 0.693147182f, p);
}

// Estimated mass of a pass-1 bin word relative to e^(c - ref), c the bin centre: the
// entries sit at fractions f_i of the bin (width w = 1/64), and
// sum e^(c + (f_i - 1/2) w - ref) ~ e^(c - ref) (n + w sum(f_i - 1/2) + n w^2 / 24).
// Bin b's centre lies (b + 1/2) / 64 - 32 from ref (up to the fp32 rounding of the grid
// offset, which scales every bin alike), so e^(c - ref) = e^((lane + 1/2)/64 - 32) e^g for
// bin 64 g + lane: one factor per lane and one per group.
__device__ __forceinline__ double nu_bin_mass(uint64_t word, double scale) {
  const double n = (double)(uint32_t)(word >> 32);
  if (n == 0.0) return 0.0;
  const double fsum = (double)(uint32_t)word * (1.0 / 256.0);
  return scale * (n + (fsum - 0.5 * n) * (1.0 / 64.0) + n * (1.0 / (64.0 * 64.0 * 24.0)));
}
__device__ __forceinline__ double nu_lane_scale(int lane) { return exp(((double)lane + 0.5) / 64.0 - 32.0); }

struct NuShared {
  double gexp[kNuGroups];  // e^g
  int coff[kMaxChunks + 1];  // the gathered collection: chunk c's entries are [coff[c], coff[c + 1])
  uint32_t ref_key, kmax, flags;
  int gsel, bsel, jp, ncoll, chunk_pick;
  int32_t last, pick;
  double target_d;
  uint64_t red64[kNuWaves];
  uint32_t red32[kNuWaves];
  double redd[kNuWaves];
};

template <int DT, bool ALIGNED, bool PEN, bool MASK>
__global__ void __launch_bounds__(kNuBlock) nucleus_kernel(Args a, NuRec* recs, uint64_t* ctr, uint32_t tag,
                                                           uint32_t spin_limit) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int U = 8 / VEC;              // 16-byte units per lane per batch
  constexpr int NQ = VEC * U;             // entries per lane per batch (8)
  constexpr int kBatchUnits = U * kWave;  // 16-byte units per batch
  constexpr int kBatchIds = kBatchUnits * VEC;
  static_assert(kBatchIds == kNuBatchIds, "512 ids per batch");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ NuShared s;
  __shared__ int s_timeout;
  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  const int S = a.S, V = a.V;

  // ---- (row, chunk) by workgroup index: a row's S workgroups are consecutive, and
  // workgroups are dispatched in index order, so when one of a row's workgroups runs, every
  // lower-indexed row has all of its workgroups running or done, and the row's others start
  // as those finish (the plan also keeps the grid within what the chip holds at once). A
  // global ticket in start order would make that independent of dispatch order, but every
  // workgroup would contend for one counter. Should a row's workgroups ever not meet, the
  // bounded waits report the row as ARBOR_ID_STALLED instead of hanging ----
  const int ticket = (int)blockIdx.x;
  const int row = ticket / S, chunk = ticket % S;
  uint64_t* bar_w = S > 1 ? ctr + row : nullptr;
  uint64_t* fail_w = S > 1 ? ctr + a.B + row : nullptr;
  if (t == 0) {
    s_timeout = 0;
    if (S > 1 && chunk == 0) {  // the row's stamp: this call's tag, nothing counted yet
      __hip_atomic_store(fail_w, (uint64_t)tag << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_all_memory();
      __hip_atomic_store(bar_w, (uint64_t)tag << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  uint32_t passed = 0u;
  bool stalled = false;
  auto sync_row = [&]() {
    nu_barrier(bar_w, fail_w, tag, ++passed * (uint32_t)S, spin_limit, &s_timeout);
    if (s_timeout) stalled = true;
  };
  const int c0 = chunk * a.chunk_len, c1 = min(V, c0 + a.chunk_len);
  const int n_units = (c1 - c0 + VEC - 1) / VEC;
  const int n_batches = (n_units + kBatchUnits - 1) / kBatchUnits;
  const NuLayout L = NuLayout::make(n_batches, PEN ? a.bitmap_words : 0, PEN ? (1 << a.hash_bits) : 0);
  uint64_t* hist = reinterpret_cast<uint64_t*>(smem);
  double* gsum = reinterpret_cast<double*>(smem + L.gsum_off);
  double* seg = reinterpret_cast<double*>(smem + L.seg_off);
  uint64_t* segx = reinterpret_cast<uint64_t*>(smem + L.segx_off);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem + L.bitmap_off);
  uint32_t* htab = reinterpret_cast<uint32_t*>(smem + L.htab_off);
  // pass 2 and the sort reuse the histogram's LDS
  uint64_t* gkey = hist;                                                  // [kNuColl]
  float* gm = reinterpret_cast<float*>(hist + kNuColl);                   // [kNuColl]
  uint16_t* idx = reinterpret_cast<uint16_t*>(gm + kNuColl);              // [kNuColl] sorted -> entry
  uint32_t* scnt = reinterpret_cast<uint32_t*>(idx + kNuColl);            // [kNuSub]
  uint32_t* sbeg = scnt + kNuSub;                                         // [kNuSub]
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = MASK ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  float* prow = a.write_probs ? a.out_probs + (size_t)row * (size_t)V : nullptr;
  NuRec* mine = S > 1 ? recs + ticket : nullptr;
  const NuRec* rowr = S > 1 ? recs + (size_t)row * (size_t)S : nullptr;

  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(xrow) + (size_t)c0 * Elem<DT>::kBytes), (short)0,
      (c1 - c0) * Elem<DT>::kBytes, 0x00020000);
  struct Batch {
    uint32_t w[U][4];
    uint32_t mw[U];
  };
  // local batch b: lane l holds units b * kBatchUnits + u * 64 + l of the chunk
  auto load = [&](int b, Batch& bt) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int unit = b * kBatchUnits + u * kWave + lane;
      if (ALIGNED) {
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, unit * 16, 0, 0);
        bt.w[u][0] = v.x;
        bt.w[u][1] = v.y;
        bt.w[u][2] = v.z;
        bt.w[u][3] = v.w;
      } else {
        load_raw<DT>(xrow, c0 + unit * VEC, c1, false, bt.w[u]);
      }
      if (MASK) bt.mw[u] = unit < n_units ? mrow[(c0 + unit * VEC) >> 5] : 0u;
    }
  };
  const bool counts = a.pen.fp != 0.0f;
  auto id_of = [&](int b, int q) { return c0 + (b * kBatchUnits + (q / VEC) * kWave + lane) * VEC + (q % VEC); };
  // final z of a batch's entries (-inf: past the chunk or masked); NaN / +inf as they are
  auto zfin = [&](int b, const Batch& bt, float* z) __attribute__((always_inline)) {
    const bool full = (b + 1) * kBatchUnits <= n_units && (ALIGNED || (b + 1) * kBatchIds <= c1 - c0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      z[q] = unpack_unit<DT>(bt.w[q / VEC], q % VEC) * a.inv_t;
      if (MASK) {
        const int id = id_of(b, q);
        if (!((bt.mw[q / VEC] >> (id & 31)) & 1u)) z[q] = -INFINITY;
      }
    }
    if (!full) {
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        if (id_of(b, q) >= c1) z[q] = -INFINITY;
    }
    if (PEN) {
      // a unit's ids share one bitmap word (units are aligned to VEC <= 8 ids); the slots
      // of history ids (bit q of hm) are penalised one at a time, rarely
      uint32_t hm = 0u;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int off = (b * kBatchUnits + u * kWave + lane) * VEC;  // chunk-relative id of the unit
        const uint32_t wbits = off < c1 - c0 ? bitmap[off >> 5] : 0u;
        hm |= ((wbits >> (off & 31)) & ((1u << VEC) - 1u)) << (u * VEC);
      }
      while (__ballot(hm != 0u)) {
        const bool pending = hm != 0u;  // lanes with no slot left take part idle
        const int qh = pending ? __builtin_ctz(hm) : 0;
        hm &= hm - 1u;
        float zq = z[0];
#pragma unroll
        for (int q = 1; q < NQ; ++q) zq = qh == q ? z[q] : zq;
        // occurrence counts matter only to a frequency penalty
        const uint32_t cnt = counts ? hist_count(htab, (uint32_t)a.hash_bits, (uint32_t)id_of(b, qh)) : 1u;
        const float zp = penalize(zq, cnt, a.pen);
        const bool act = pending && cnt != 0u;
#pragma unroll
        for (int q = 0; q < NQ; ++q) z[q] = act && qh == q ? zp : z[q];
      }
    }
  };

  // ---- set-up: the anchor's ids (wave 0) and the first batches are requested, the LDS
  // cleared, the history inserted ----
  uint32_t aw[U][4], amw[U];
  if (wave == 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e0 = (u * kWave + lane) * VEC;
      load_raw<DT>(xrow, e0, V, a.aligned && V % VEC == 0, aw[u]);
      amw[u] = MASK && e0 < V ? mrow[e0 >> 5] : ~0u;
    }
  }
  Batch b0, b1, b2;
  int i0 = wave, i1 = wave + kNuWaves, i2 = wave + 2 * kNuWaves;
  load(i0, b0);
  load(i1, b1);
  load(i2, b2);
  for (int i = t; i < kNuBins; i += kNuBlock) hist[i] = 0ull;
  for (int i = t; i < n_batches; i += kNuBlock) {
    seg[i] = 0.0;
    segx[i] = 0ull;
  }
  if (PEN) {
    for (int i = t; i < a.bitmap_words; i += kNuBlock) bitmap[i] = 0u;
    for (int i = t; i < (1 << a.hash_bits); i += kNuBlock) htab[i] = kEmptySlot;
  }
  if (t == 0) {
    s.ref_key = 0u;
    s.kmax = 0u;
    s.flags = 0u;
    s.gsel = -1;
    s.bsel = -1;
    s.jp = -1;
    s.ncoll = 0;
    s.chunk_pick = -1;
    s.last = -1;
    s.pick = -1;
  }
  __syncthreads();
  uint32_t flags = 0u;
  if (PEN) {
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    for (int j = t; j < a.H; j += kNuBlock) {
      const int32_t id = h[j];
      if (id < 0) continue;
      if (id >= V) {
        flags |= kFlagBadHistory;
      } else {
        hist_insert(htab, (uint32_t)a.hash_bits, (uint32_t)id);
        if (id >= c0 && id < c1) atomicOr(&bitmap[(id - c0) >> 5], 1u << ((id - c0) & 31));
      }
    }
  }
  __syncthreads();

  // ---- the grid's anchor: the largest tempered logit of the row's first 512 ids (its
  // loads were issued first), the same in every workgroup of the row. Penalties are left
  // out: the grid reaches 96 above the anchor, and an entry beyond it only sends the row to
  // the exact solver ----
  if (wave == 0) {
    uint32_t km = 0u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e0 = (u * kWave + lane) * VEC;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int id = e0 + j;
        const float z = unpack_unit<DT>(aw[u], j) * a.inv_t + 0.0f;
        if (id < V && ((amw[u] >> (id & 31)) & 1u) && z != -INFINITY && !is_invalid(z)) km = max(km, order_key(z));
      }
    }
    km = wave_max(km);
    if (lane == 0) s.ref_key = km;
  }
  __syncthreads();
  // no finite value there (masked rows): the grid is anchored at 0; an entry beyond it
  // sends the row to the exact solver
  const float ref = s.ref_key ? key_value(s.ref_key) : 0.0f;
  const float glo = ref - kNuBelow;
  const float yoff = -glo * kNuScale;  // y = fma(z, 64, yoff): the bin coordinate of z

  // ---- 1. pass 1 ----
  float zmx = -INFINITY;
  bool over = false, bad = false;
  auto pass1 = [&](int b, const Batch& bt) __attribute__((always_inline)) {
    float z[NQ];
    zfin(b, bt, z);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      bad |= is_invalid(z[q]);
      zmx = fmaxf(zmx, z[q]);
      const float y = __builtin_fmaf(z[q], kNuScale, yoff);
      over |= y >= (float)kNuBins;
      const float yc = fminf(fmaxf(y, 0.0f), (float)kNuBins - 0.001f);
      const int bin = (int)yc;
      const uint32_t fr = (uint32_t)(__builtin_amdgcn_fractf(yc) * 256.0f);
      if (z[q] != -INFINITY)
        atomicAdd(reinterpret_cast<unsigned long long*>(hist + bin),
                  (unsigned long long)((1ull << 32) | (uint64_t)fr));
    }
  };
  for (;;) {
    if (i0 >= n_batches) break;
    pass1(i0, b0);
    i0 += 3 * kNuWaves;
    load(i0, b0);
    if (i1 >= n_batches) break;
    pass1(i1, b1);
    i1 += 3 * kNuWaves;
    load(i1, b1);
    if (i2 >= n_batches) break;
    pass1(i2, b2);
    i2 += 3 * kNuWaves;
    load(i2, b2);
  }
  // pass 2's first batches are requested now: they arrive while the cut bin is found
  load(wave, b0);
  load(wave + kNuWaves, b1);
  load(wave + 2 * kNuWaves, b2);
  if (bad) flags |= kFlagInvalid;
  if (over) flags |= kNuFlagFallback;
  {
    const uint32_t fw = wave_reduce(flags, [](uint32_t x, uint32_t y) { return x | y; });
    const uint32_t kw = wave_max(zmx > -INFINITY ? order_key(zmx + 0.0f) : 0u);
    if (lane == 0) {
      if (fw) atomicOr(&s.flags, fw);
      if (kw) atomicMax(&s.kmax, kw);
    }
  }
  __syncthreads();
  // the chunk's group sums (wave w: groups w, w + 16, ...; lane l: bin 64 g + l)
  {
    // e^g for the wave's groups g = wave + 16 k: e^wave, then factors of e^16
    const double lscale = nu_lane_scale(lane);
    double ge = exp((double)wave);
    for (int g = wave; g < kNuGroups; g += kNuWaves) {
      if (lane == 0) s.gexp[g] = ge;
      const double m = wave_sum(nu_bin_mass(hist[g * kWave + lane], lscale * ge));
      if (lane == 0) gsum[g] = m;
      ge *= 8886110.520507872;  // e^16
    }
  }
  __syncthreads();
  const bool use_min_p = a.min_p > 0.0f;
  const bool use_top_p = a.top_p < 1.0f;
  uint32_t kmax;
  if (S > 1) {
    if (t == 0) {
      pub_store(&mine->kmax, s.kmax);
      pub_store(&mine->flags, s.flags);
    }
    for (int g = t; g < kNuGroups; g += kNuBlock) pub_store(&mine->gsum[g], gsum[g]);
    sync_row();  // B1
    // lane c reads chunk c's record (S <= 64): one round trip instead of S
    uint32_t km = 0u, fl = 0u;
    if (lane < S) {
      km = pub_load(&rowr[lane].kmax);
      fl = pub_load(&rowr[lane].flags);
    }
    kmax = wave_max(km);
    flags = wave_reduce(fl, [](uint32_t x, uint32_t y) { return x | y; });
  } else {
    kmax = s.kmax;
    flags = s.flags;
  }
  if (stalled) {
    // a barrier gave up: arrive at the rest so the row's counts stay whole, then report
    sync_row();
    sync_row();
    if (t == 0) __hip_atomic_exchange(a.out_ids + row, ARBOR_ID_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if ((flags & (kFlagBadHistory | kFlagInvalid)) || kmax == 0u) {
    // the same decision in every workgroup of the row: none meets a later barrier
    if (chunk == 0 && t == 0)
      a.out_ids[row] = (flags & kFlagBadHistory) ? ARBOR_ID_BAD_HISTORY
                                                  : ((flags & kFlagInvalid) ? ARBOR_ID_INVALID : ARBOR_ID_EMPTY);
    if (prow)
      for (int i = c0 + t; i < c1; i += kNuBlock) prow[i] = 0.0f;
    return;
  }
  if (flags & kNuFlagFallback) {
    if (chunk == 0) solve_row<kNuBlock, DT>(a, row, htab, *reinterpret_cast<SolverShared*>(smem));
    return;
  }
  const float zmax = key_value(kmax);

  // ---- the estimated cut bin: top-p group then bin, from the row's group sums ----
  if (use_top_p) {
    if (wave == 0) {
      // lane l: groups 127 - 2l and 126 - 2l (descending)
      double gm0 = 0.0, gm1 = 0.0;
      const int g0 = kNuGroups - 1 - 2 * lane, g1 = g0 - 1;
      if (S > 1) {
        for (int cb = 0; cb < S; cb += 4) {
          double x0[4], x1[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            x0[j] = cb + j < S ? pub_load(&rowr[cb + j].gsum[g0]) : 0.0;
            x1[j] = cb + j < S ? pub_load(&rowr[cb + j].gsum[g1]) : 0.0;
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (cb + j < S) {
              gm0 += x0[j];
              gm1 += x1[j];
            }
          }
        }
      } else {
        gm0 = gsum[g0];
        gm1 = gsum[g1];
      }
      const double pair = gm0 + gm1;
      const double incl = wave_scan_incl(pair);
      const double tot = lane_get(incl, kWave - 1);
      const double target = (double)a.top_p * tot;
      const uint64_t hit = __ballot(incl >= target);
      int gsel = -1;
      double before = 0.0;
      if (hit) {
        const int l = __ffsll((long long)hit) - 1;
        const double ex = lane_get(incl - pair, l);
        const double m0 = lane_get(gm0, l);
        gsel = ex + m0 >= target ? kNuGroups - 1 - 2 * l : kNuGroups - 2 - 2 * l;
        before = ex + m0 >= target ? ex : ex + m0;
      }
      if (lane == 0) {
        s.gsel = gsel;
        s.target_d = target - before;  // mass still to reach inside the selected group
      }
    }
    __syncthreads();
    const int gsel = s.gsel;
    if (S > 1) {
      if (gsel >= 0)
        for (int i = t; i < kWave; i += kNuBlock) pub_store(&mine->gbins[i], hist[gsel * kWave + i]);
      sync_row();  // B1b
      if (stalled) {
        sync_row();
        if (t == 0) __hip_atomic_exchange(a.out_ids + row, ARBOR_ID_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
    }
    if (wave == 0 && gsel >= 0) {
      // lane l: bin 64 g + 63 - l (descending), its words summed over the row's chunks
      const int bin = gsel * kWave + kWave - 1 - lane;
      uint64_t wsum = 0ull;
      if (S > 1) {
        for (int cb = 0; cb < S; cb += 4) {
          uint64_t x[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) x[j] = cb + j < S ? pub_load(&rowr[cb + j].gbins[kWave - 1 - lane]) : 0ull;
#pragma unroll
          for (int j = 0; j < 4; ++j) wsum += x[j];
        }
      } else {
        wsum = hist[bin];
      }
      const double m = nu_bin_mass(wsum, nu_lane_scale(kWave - 1 - lane) * s.gexp[gsel]);
      const double incl = wave_scan_incl(m);
      const uint64_t hit = __ballot(incl >= s.target_d);
      // not reached inside the group (rounding): its lowest bin
      const int l = hit ? __ffsll((long long)hit) - 1 : kWave - 1;
      if (lane == 0) s.bsel = gsel * kWave + kWave - 1 - l;
    }
    __syncthreads();
  }
  int bcut = use_top_p ? s.bsel : -1;
  if (use_top_p && bcut < 0) bcut = 0;  // nothing reached (all mass below the grid): keep from the bottom
  // when min-p's edge lies above the top-p estimate by more than a bin, min-p decides the
  // kept set and top-p keeps every collected entry (its cut lies below them)
  bool minp_range = false;
  if (use_min_p) {
    const float ym = __builtin_fmaf((float)((double)zmax + log((double)a.min_p)), kNuScale, yoff);
    const int bm = (int)fminf(fmaxf(ym, 0.0f), (float)kNuBins - 0.001f);
    minp_range = bm > bcut + 1;
    bcut = max(bcut, bm);
  }
  // bins above bhi are kept whatever the exact cut, bins below blo are not
  const bool has_cut = use_top_p || use_min_p;
  const float ykeep = has_cut ? (float)(bcut + 2) : -1.0f;  // y >= ykeep: kept
  const float ycoll = has_cut ? (float)(bcut - 1) : -1.0f;  // ycoll <= y < ykeep: collected

  // ---- 2. pass 2 ----
  __syncthreads();  // every wave is done with the histogram: the collection reuses it
  if (t == 0) s.ncoll = 0;
  __syncthreads();
  double E = 0.0;
  int32_t last = -1;
  bool minp_bad = false;
  {
    int j0 = wave, j1 = wave + kNuWaves, j2 = wave + 2 * kNuWaves;  // requested after pass 1
    auto pass2 = [&](int b, const Batch& bt) __attribute__((always_inline)) {
      float z[NQ], e[NQ];
      zfin(b, bt, z);
      double sk = 0.0;
      uint32_t cbits = 0u;  // slots to collect
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        z[q] = z[q] + 0.0f;
        const bool fin = z[q] != -INFINITY;
        const float y = __builtin_fmaf(z[q], kNuScale, yoff);
        const bool keep = fin && y >= ykeep;
        const bool coll = fin && !keep && y >= ycoll;
        e[q] = nu_exp(z[q], zmax);
        const double ed = fin ? (double)e[q] : 0.0;
        E += ed;
        sk += keep ? ed : 0.0;
        last = keep ? max(last, id_of(b, q)) : last;
        if (use_min_p && keep && !(e[q] >= a.min_p)) minp_bad = true;
        cbits |= coll ? 1u << q : 0u;
      }
      // the batch's collected slots: one slot reservation for the whole wave
      const int nmine = __builtin_popcount(cbits);
      if (__ballot(nmine != 0)) {
        const int incl = wave_scan_incl(nmine);
        int base = 0;
        if (lane == kWave - 1) base = atomicAdd(&s.ncoll, incl);
        base = lane_get(base, kWave - 1) + incl - nmine;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          if ((cbits >> q) & 1u) {
            if (base < kNuCollChunk) {
              gkey[base] = composite(z[q], id_of(b, q));
              gm[base] = e[q];
            }
            ++base;
          }
        }
      }
      sk = wave_sum(sk);
      if (lane == 0) seg[b] = sk;
    };
    for (;;) {
      if (j0 >= n_batches) break;
      pass2(j0, b0);
      j0 += 3 * kNuWaves;
      load(j0, b0);
      if (j1 >= n_batches) break;
      pass2(j1, b1);
      j1 += 3 * kNuWaves;
      load(j1, b1);
      if (j2 >= n_batches) break;
      pass2(j2, b2);
      j2 += 3 * kNuWaves;
      load(j2, b2);
    }
  }
  {
    // the chunk's totals, in a fixed order: lanes, then waves
    const double Ew = wave_sum(E);
    const int32_t lw = wave_max(last);
    const bool mb = __ballot(minp_bad) != 0ull;
    if (lane == 0) {
      s.redd[wave] = Ew;
      s.red32[wave] = (uint32_t)(lw + 1);
      if (mb) atomicOr(&s.flags, kNuFlagFallback);
    }
  }
  __syncthreads();
  double Ec = 0.0, above_c = 0.0;
  int32_t last_c = -1;
  for (int w = 0; w < kNuWaves; ++w) {
    Ec += s.redd[w];
    last_c = max(last_c, (int32_t)s.red32[w] - 1);
  }
  for (int b = 0; b < n_batches; ++b) above_c += seg[b];
  const int ncoll_c = s.ncoll;
  uint32_t flags_c = s.flags | (ncoll_c > kNuCollChunk ? kNuFlagFallback : 0u);
  __syncthreads();

  // ---- 3. the collected entries of the row, sorted; the exact cut ----
  double Erow = Ec, above = above_c;
  int32_t last_row = last_c;
  int n = min(ncoll_c, kNuCollChunk);
  if (S > 1) {
    if (t == 0) {
      pub_store(&mine->E, Ec);
      pub_store(&mine->above, above_c);
      pub_store(&mine->last, last_c);
      pub_store(&mine->ncoll, ncoll_c);
      pub_store(&mine->flags, flags_c);
    }
    for (int i = t; i < n; i += kNuBlock) {
      pub_store(&mine->ckey[i], gkey[i]);
      pub_store(&mine->cm[i], gm[i]);
    }
    sync_row();  // B2
    if (stalled) {
      if (t == 0) __hip_atomic_exchange(a.out_ids + row, ARBOR_ID_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    Erow = 0.0;
    above = 0.0;
    last_row = -1;
    flags_c = 0u;
    n = 0;
    for (int cb = 0; cb < S; cb += 4) {
      // the records of up to 4 chunks in flight, combined in chunk order
      double xe[4], xa[4];
      int32_t xl[4], xn[4];
      uint32_t xf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = cb + j < S;
        xe[j] = in ? pub_load(&rowr[cb + j].E) : 0.0;
        xa[j] = in ? pub_load(&rowr[cb + j].above) : 0.0;
        xl[j] = in ? pub_load(&rowr[cb + j].last) : -1;
        xf[j] = in ? pub_load(&rowr[cb + j].flags) : 0u;
        xn[j] = in ? pub_load(&rowr[cb + j].ncoll) : 0;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (cb + j >= S) break;
        Erow += xe[j];
        above += xa[j];
        last_row = max(last_row, xl[j]);
        flags_c |= xf[j];
        const int nc = xn[j];
        if (t == 0) s.coff[cb + j] = n;
        if (nc > kNuCollChunk || n + nc > kNuColl) flags_c |= kNuFlagFallback;
        n = min(n + min(nc, kNuCollChunk), kNuColl);
      }
    }
    if (!(flags_c & kNuFlagFallback)) {
      // every entry at once: entry i of the row belongs to the chunk whose range holds it
      __syncthreads();
      static_assert(kNuColl == 4 * kNuBlock, "four collected entries per thread");
      uint64_t xk[4];
      float xm[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = t + j * kNuBlock;
        xk[j] = 0ull;
        xm[j] = 0.0f;
        if (i < n) {
          int c = 0;
          while (c + 1 < S && s.coff[c + 1] <= i) ++c;
          xk[j] = pub_load(&rowr[c].ckey[i - s.coff[c]]);
          xm[j] = pub_load(&rowr[c].cm[i - s.coff[c]]);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = t + j * kNuBlock;
        if (i < n) {
          gkey[i] = xk[j];
          gm[i] = xm[j];
        }
      }
    }
    if (t == 0) s.coff[S] = n;
    __syncthreads();
  } else {
    if (t == 0) {
      s.coff[0] = 0;
      s.coff[1] = n;
    }
    __syncthreads();
  }
  // counting sort by sub-bin (descending), then insertion sorts inside the sub-bins
  if (!(flags_c & kNuFlagFallback) && has_cut && n > 0) {
    scnt[t] = 0u;
    __syncthreads();
    const float sub_scale = (float)kNuSub / 3.0f;
    auto sub_of = [&](uint64_t key) -> int {
      const float y = __builtin_fmaf(composite_z(key), kNuScale, yoff);
      const int sb = (int)fminf(fmaxf((y - ycoll) * sub_scale, 0.0f), (float)kNuSub - 0.001f);
      return kNuSub - 1 - sb;  // descending z
    };
    for (int i = t; i < n; i += kNuBlock) atomicAdd(&scnt[sub_of(gkey[i])], 1u);
    __syncthreads();
    const uint32_t cnt = scnt[t];
    uint32_t tot;
    const uint32_t beg = block_scan_excl<kNuBlock, uint32_t>(cnt, s.red32, &tot);
    sbeg[t] = beg;
    const bool wide = __syncthreads_or(cnt > (uint32_t)kNuSubMax);
    if (wide) {
      flags_c |= kNuFlagFallback;  // heavy ties: the exact solver
    } else {
      for (int i = t; i < n; i += kNuBlock) idx[atomicAdd(&sbeg[sub_of(gkey[i])], 1u)] = (uint16_t)i;
      __syncthreads();
      // sub-bin t holds positions [beg, beg + cnt)
      for (int i = 1; i < (int)cnt; ++i) {
        const uint16_t v = idx[beg + i];
        const uint64_t kv = gkey[v];
        int j = i - 1;
        while (j >= 0 && gkey[idx[beg + j]] < kv) {
          idx[beg + j + 1] = idx[beg + j];
          --j;
        }
        idx[beg + j + 1] = v;
      }
      __syncthreads();
    }
  }
  uint64_t cut_key = 0ull;  // kept iff composite >= cut_key (top-p), and e >= min_p
  if (!(flags_c & kNuFlagFallback) && use_top_p) {
    const double tgt = (double)a.top_p * Erow;
    // running mass over the sorted entries, 4 per thread (n <= 4096)
    double m4[4], loc = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = t * 4 + j;
      m4[j] = i < n ? (double)gm[idx[i]] : 0.0;
      loc += m4[j];
    }
    double tot;
    const double ex = block_scan_excl<kNuBlock, double>(loc, s.redd, &tot);
    if (t == 0) s.jp = -1;
    __syncthreads();
    if (above < tgt && above + tot >= tgt && above + ex < tgt && above + ex + loc >= tgt) {
      double run = above + ex;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        run += m4[j];
        if (run >= tgt) {
          s.jp = t * 4 + j;
          break;
        }
      }
    }
    __syncthreads();
    int jp = s.jp;
    if (jp < 0 && minp_range && above < tgt && above + tot < tgt) jp = n;  // below the range: keep all
    if (jp < 0) flags_c |= kNuFlagFallback;  // the cut lies outside the collected bins
    else cut_key = jp < n ? gkey[idx[jp]] : 0ull;
  }
  if (flags_c & kNuFlagFallback) {
    if (chunk == 0) solve_row<kNuBlock, DT>(a, row, htab, *reinterpret_cast<SolverShared*>(smem));
    return;
  }
  auto kept_coll = [&](int i) -> bool {
    return gkey[i] >= cut_key && (!use_min_p || gm[i] >= a.min_p);
  };

  // ---- 4. the draw ----
  // kept mass of each chunk: its surely kept entries plus its kept collected ones (the
  // gathered entries of chunk c are [coff[c], coff[c + 1])), summed in a fixed order
  double kept_mass = 0.0;   // of the whole row
  double before = 0.0;      // of the chunks before this one
  double mine_mass = 0.0;   // of this chunk
  int32_t lastk = last_row;  // the row's largest kept id
  int32_t last_mine = -1;    // this chunk's largest kept id
  {
    if (wave == 0) {
      double acc_before = 0.0, acc_all = 0.0, acc_mine = 0.0;
      int32_t lk = -1, lkm = -1;
      // lane c holds chunk c's mass above the collected bins and largest kept id (S <= 64)
      double abv = 0.0;
      int32_t lst = -1;
      if (S > 1 && lane < S) {
        abv = pub_load(&rowr[lane].above);
        lst = pub_load(&rowr[lane].last);
      }
      for (int c = 0; c < S; ++c) {
        double cm = 0.0;
        int32_t lc = -1;
        for (int i = s.coff[c] + lane; i - lane < s.coff[c + 1]; i += kWave) {
          double v = 0.0;
          if (i < s.coff[c + 1] && kept_coll(i)) {
            v = (double)gm[i];
            lc = max(lc, composite_id(gkey[i]));
          }
          cm += wave_sum(v);
        }
        lc = wave_max(lc);
        const double ck = (S > 1 ? lane_get(abv, c) : above_c) + cm;
        if (c < chunk) acc_before += ck;
        if (c == chunk) {
          acc_mine = ck;
          lkm = max(lc, S > 1 ? lane_get(lst, c) : last_c);
        }
        acc_all += ck;
        lk = max(lk, lc);
      }
      if (lane == 0) {
        s.redd[0] = acc_all;
        s.redd[1] = acc_before;
        s.redd[2] = acc_mine;
        s.last = max(last_row, lk);
        s.pick = lkm;
      }
    }
    __syncthreads();
    kept_mass = s.redd[0];
    before = s.redd[1];
    mine_mass = s.redd[2];
    lastk = s.last;
    last_mine = s.pick;
    __syncthreads();
  }
  const double target = (double)a.uniforms[row] * kept_mass;
  const bool crossing = before <= target && target < before + mine_mass;
  // kept test and mass of any entry of this chunk (the decisions pass 2 and the cut made)
  auto kept_any = [&](float zq, int id, float* e) -> bool {
    if (zq == -INFINITY) return false;
    const float y = __builtin_fmaf(zq, kNuScale, yoff);
    if (y < ycoll) return false;
    *e = nu_exp(zq, zmax);
    if (y < ykeep) {
      if (composite(zq, id) < cut_key || (use_min_p && !(*e >= a.min_p))) return false;
    }
    return true;
  };
  if (crossing) {
    // this chunk's kept collected entries join their batches (fixed point: exact, any order)
    for (int i = t; i < n; i += kNuBlock) {
      const int id = composite_id(gkey[i]);
      if (id >= c0 && id < c1 && kept_coll(i))
        atomicAdd(reinterpret_cast<unsigned long long*>(&segx[(id - c0) / kBatchIds]),
                  (unsigned long long)mass_fixed(gm[i]));
    }
    __syncthreads();
    if (wave == 0) {
      double run = before;
      int bs = -1;
      for (int bb = 0; bb < n_batches; bb += kWave) {
        const double v =
            bb + lane < n_batches ? seg[bb + lane] + (double)segx[bb + lane] * (1.0 / (double)kMassScale) : 0.0;
        const double incl = run + wave_scan_incl(v);
        const uint64_t hit = __ballot(incl > target);
        if (hit) {
          const int l = __ffsll((long long)hit) - 1;
          bs = bb + l;
          run = lane_get(incl - v, l);
          break;
        }
        run = lane_get(incl, kWave - 1);
      }
      int32_t pick = last_mine;  // no batch reached (rounding): the chunk's last kept id
      if (bs >= 0) {
        Batch bt;
        load(bs, bt);
        float z[NQ];
        zfin(bs, bt, z);
        float e[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          e[q] = 0.0f;
          if (!kept_any(z[q] + 0.0f, id_of(bs, q), &e[q])) e[q] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          double lw = 0.0;
#pragma unroll
          for (int j = 0; j < VEC; ++j) lw += (double)e[u * VEC + j];
          const double incl = run + wave_scan_incl(lw);
          const uint64_t hit = __ballot(incl > target);
          if (hit) {
            const int l = __ffsll((long long)hit) - 1;
            int32_t p = -1, lastw = -1;
            if (lane == l) {
              double acc = incl - lw;
#pragma unroll
              for (int j = 0; j < VEC; ++j) {
                const float ej = e[u * VEC + j];
                acc += (double)ej;
                if (ej > 0.0f) lastw = id_of(bs, u * VEC + j);
                if (p < 0 && ej > 0.0f && acc > target) p = id_of(bs, u * VEC + j);
              }
              if (p < 0) p = lastw;  // rounding inside the lane: its last kept id
            }
            pick = lane_get(p, l);
            break;
          }
          run = lane_get(incl, kWave - 1);
        }
      }
      if (lane == 0) s.pick = pick;
    }
    __syncthreads();
    if (t == 0) {
      if (S > 1) {
        store_row_id(a.out_ids + row, s.pick);
      } else {
        a.out_ids[row] = s.pick;
        ring_append(a, row, s.pick);  // one workgroup: the row's history was read at the start
      }
    }
  } else if (!(target < kept_mass) && lastk >= c0 && lastk < c1) {
    // no crossing (u * E rounds to E, or u is NaN): the last kept id, by its chunk
    if (t == 0) {
      if (S > 1) {
        store_row_id(a.out_ids + row, lastk);
      } else {
        a.out_ids[row] = lastk;
        ring_append(a, row, lastk);
      }
    }
  }
  if (prow) {
    const double Ed = kept_mass;
    for (int b = wave; b < n_batches; b += kNuWaves) {
      Batch bt;
      load(b, bt);
      float z[NQ];
      zfin(b, bt, z);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int id = id_of(b, q);
        if (id >= c1) continue;
        float e = 0.0f;
        prow[id] = kept_any(z[q] + 0.0f, id, &e) ? (float)((double)e / Ed) : 0.0f;
      }
    }
  }
}

}  // namespace arbor
