// sampling.hip -- MI355X (gfx950) token-sampling kernels and the extern "C" ABI of
// libarbor_hip.so (declared in include/arbor_sampling.h).
//
// Two device paths compute the same contract:
//
//  * stream_kernel  (top-k <= 256, or min-p as the only filter): each row is split into
//    S chunks; one 256-thread workgroup streams one chunk from HBM exactly once with
//    16-byte loads, applies temperature / penalties (LDS history table) / allow-mask, and
//    keeps per-wave candidate lists in LDS. A candidate list is pruned by an exact
//    wave-level radix select whenever it fills, so a wave only ever holds the top-k (or
//    the min-p band) of what it has seen. Each chunk publishes a sorted list; the last
//    workgroup of a row to arrive (atomic arrival counter) merges the S lists
//    (merge-path ranks) and applies top-k, top-p, min-p and the inverse-CDF draw in fp64
//    on at most 1024 candidates. No tempered logit is ever written back to HBM.
//
//  * row solver  (top-p without top-k, plain sampling, or a stream row whose candidate
//    list overflowed): one workgroup per row materialises z in the workspace and finds
//    each cut with an MSB-first radix select on the 64-bit rank key, weighting by count
//    (top-k) or by probability mass (top-p), then draws with a block scan in id order.
//    Mass is fixed point (2^-40) so every sum is exact and order independent.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <cmath>

#include "../../include/arbor_sampling.h"
#include "device_common.hpp"

namespace arbor {

constexpr int kStreamBlock = 256;
constexpr int kStreamWaves = kStreamBlock / kWave;
constexpr int kWaveCap = 1024;     // candidates a wave holds in LDS
constexpr int kChunkSlot = 256;    // candidates a chunk publishes
constexpr int kFinalCap = 1024;    // candidates the finishing workgroup merges
constexpr int kMaxTopK = 256;      // largest top-k of the streaming path
constexpr int kUnroll = 4;         // 16-byte loads in flight per lane
constexpr int kSolverBlock = 1024;
constexpr int kMaxChunks = 64;

struct Args {
  const void* logits;
  int64_t ld;
  int V, B;
  const int32_t* hist;
  int H;
  const uint32_t* mask;
  int mask_words;
  const float* uniforms;
  int32_t* out_ids;
  float* out_probs;
  float inv_t;
  Penalty pen;
  int top_k;     // 0 = off (already clamped: k >= V means off)
  float top_p;   // 1 = off
  float min_p;   // 0 = off
  float ln_min_p_lo;  // ln(min_p) minus a safety margin, candidate band of min-p
  int S, chunk_len, chunk_cap;
  int hash_bits, bitmap_words;
  int aligned, xcd_map, write_probs;
  uint32_t* counters;  // [B]      arrival counters, zero between calls
  uint32_t* hdr;       // [B*S*4]  count, flags
  uint64_t* cand;      // [B*S*kChunkSlot] sorted composites per chunk
  float* zbuf;         // [B*V]    row solver's tempered logits
};

// ---------------------------------------------------------------------------------------
// Element loads
// ---------------------------------------------------------------------------------------
template <int DT>
struct Elem;
template <>
struct Elem<ARBOR_DTYPE_F32> {
  static constexpr int kVec = 4;
  static __device__ __forceinline__ float one(const void* base, int64_t i) {
    return static_cast<const float*>(base)[i];
  }
  static __device__ __forceinline__ void vec(const void* base, int64_t i, float* x) {
    const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  }
};
template <>
struct Elem<ARBOR_DTYPE_BF16> {
  static constexpr int kVec = 8;
  static __device__ __forceinline__ float one(const void* base, int64_t i) {
    return bf16_bits_to_float(static_cast<const uint16_t*>(base)[i]);
  }
  static __device__ __forceinline__ void vec(const void* base, int64_t i, float* x) {
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = __uint_as_float(w[j] << 16);
      x[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
    }
  }
};

// VEC elements starting at e0 of a row; positions at or beyond `end` read as -inf.
template <int DT>
__device__ __forceinline__ void load_unit(const void* row, int e0, int end, bool aligned, float* x) {
  constexpr int VEC = Elem<DT>::kVec;
  if (aligned && e0 + VEC <= end) {
    Elem<DT>::vec(row, e0, x);
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) x[j] = e0 + j < end ? Elem<DT>::one(row, e0 + j) : -INFINITY;
  }
}

__device__ __forceinline__ const void* row_ptr(const Args& a, int dtype_size, int row) {
  return static_cast<const char*>(a.logits) + (size_t)row * (size_t)a.ld * (size_t)dtype_size;
}

// ---------------------------------------------------------------------------------------
// Wave-level candidate maintenance (buffer of composites in LDS, wave-private)
// ---------------------------------------------------------------------------------------

// Acceptance threshold that keeps every entry of the buffer (used only on a broken
// invariant, so that a wave can never read a lane index of -1).
__device__ __forceinline__ float thr_unchanged_keep_all(const uint64_t* buf, int n) {
  uint64_t mn = ~0ull;
  for (int i = lane_id(); i < n; i += kWave) mn = buf[i] < mn ? buf[i] : mn;
  mn = wave_min(mn);
  return n > 0 ? composite_z(mn) - 1.0f : -INFINITY;
}

// Keep exactly the k best of n entries (n > k). Returns the z value of the k-th best,
// the strict acceptance threshold for everything this wave sees later (later ids are
// larger, so an equal z loses the tie).
__device__ float wave_keep_topk(uint64_t* buf, int& n, int k, uint32_t* hist) {
  const int lane = lane_id();
  uint64_t lo = ~0ull, hi = 0;
  for (int i = lane; i < n; i += kWave) {
    const uint64_t c = buf[i];
    lo = c < lo ? c : lo;
    hi = c > hi ? c : hi;
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  const int hb = 63 - __clzll(hi ^ lo);
  int shift = (hb >> 3) << 3;
  uint64_t pmask = shift + 8 >= 64 ? 0ull : (~0ull << (shift + 8));
  uint64_t prefix = hi & pmask;
  uint32_t need = (uint32_t)k;
  for (;;) {
    for (int b = lane; b < 256; b += kWave) hist[b] = 0u;
    wave_lds_sync();
    for (int i = lane; i < n; i += kWave) {
      const uint64_t c = buf[i];
      if ((c & pmask) == prefix) atomicAdd(&hist[(uint32_t)(c >> shift) & 255u], 1u);
    }
    wave_lds_sync();
    uint32_t cnt[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      cnt[j] = hist[255 - 4 * lane - j];
      s += cnt[j];
    }
    wave_lds_sync();
    uint32_t run = wave_scan_incl(s) - s;
    int dsel = -1;
    uint32_t above = 0, csel = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (dsel < 0 && run < need && run + cnt[j] >= need) {
        dsel = 255 - 4 * lane - j;
        above = run;
        csel = cnt[j];
      }
      run += cnt[j];
    }
    const uint64_t bal = __ballot(dsel >= 0);
    if (bal == 0ull) return thr_unchanged_keep_all(buf, n);  // unreachable: need <= matching count
    const int src = __ffsll((long long)bal) - 1;
    dsel = __shfl(dsel, src);
    above = __shfl(above, src);
    csel = __shfl(csel, src);
    need -= above;
    prefix |= (uint64_t)dsel << shift;
    pmask |= 255ull << shift;
    if (need == csel || shift == 0) break;
    shift -= 8;
  }
  // keep every composite >= prefix (the selected bin and everything above it)
  uint64_t v[kWaveCap / kWave];
#pragma unroll
  for (int r = 0; r < kWaveCap / kWave; ++r) {
    const int i = r * kWave + lane;
    v[r] = i < n ? buf[i] : 0ull;
  }
  wave_lds_sync();
  int nn = 0;
  uint64_t mn = ~0ull;
#pragma unroll
  for (int r = 0; r < kWaveCap / kWave; ++r) {
    const bool keep = v[r] >= prefix && v[r] != 0ull;
    const uint64_t bal = __ballot(keep);
    if (keep) {
      buf[nn + lanes_below(bal)] = v[r];
      mn = v[r] < mn ? v[r] : mn;
    }
    nn += __popcll(bal);
  }
  wave_lds_sync();
  n = nn;
  return composite_z(wave_min(mn));
}

// Keep the entries with z >= (largest z) + band, band < 0 (min-p candidate band).
// Returns the new acceptance threshold.
__device__ float wave_keep_band(uint64_t* buf, int& n, float band) {
  const int lane = lane_id();
  uint64_t hi = 0;
  for (int i = lane; i < n; i += kWave) {
    const uint64_t c = buf[i];
    hi = c > hi ? c : hi;
  }
  hi = wave_max(hi);
  const float thr = composite_z(hi) + band;
  uint64_t v[kWaveCap / kWave];
#pragma unroll
  for (int r = 0; r < kWaveCap / kWave; ++r) {
    const int i = r * kWave + lane;
    v[r] = i < n ? buf[i] : 0ull;
  }
  wave_lds_sync();
  int nn = 0;
#pragma unroll
  for (int r = 0; r < kWaveCap / kWave; ++r) {
    const bool keep = v[r] != 0ull && composite_z(v[r]) >= thr;
    const uint64_t bal = __ballot(keep);
    if (keep) buf[nn + lanes_below(bal)] = v[r];
    nn += __popcll(bal);
  }
  wave_lds_sync();
  n = nn;
  return thr;
}

// Sort 64 composites held one per lane, descending (bitonic network over shuffles).
__device__ __forceinline__ uint64_t wave_sort64_desc(uint64_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t w = __shfl_xor(v, stride);
      const bool asc = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      const uint64_t mx = v > w ? v : w, mn = v > w ? w : v;
      v = (lower == asc) ? mx : mn;
    }
  }
  return v;
}

// Sort n <= kWaveCap composites of a wave buffer descending.
__device__ void wave_sort_desc(uint64_t* buf, int n) {
  const int lane = lane_id();
  if (n <= 1) return;
  if (n <= kWave) {
    uint64_t v = lane < n ? buf[lane] : 0ull;
    v = wave_sort64_desc(v);
    wave_lds_sync();
    if (lane < n) buf[lane] = v;
    wave_lds_sync();
    return;
  }
  // rank by counting (n <= 256 in practice)
  constexpr int R = kWaveCap / kWave;
  uint64_t v[R];
  int rank[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWave + lane;
    v[r] = i < n ? buf[i] : 0ull;
    rank[r] = 0;
  }
  const int rmax = (n + kWave - 1) / kWave;
  for (int j = 0; j < n; ++j) {
    const uint64_t c = buf[j];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r < rmax) rank[r] += c > v[r] ? 1 : 0;
  }
  wave_lds_sync();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r * kWave + lane < n) buf[rank[r]] = v[r];
  wave_lds_sync();
}

// Number of entries of a descending list greater than v.
__device__ __forceinline__ int count_greater(const uint64_t* list, int n, uint64_t v) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (list[mid] > v)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// Merge nl descending lists (list l = src + off[l], cnt[l] entries) by merge-path ranks:
// entry v of list l lands at out[pos_in_l + sum over other lists of count_greater].
// Entries of rank >= kout are dropped. Call with every thread of the block.
template <int BLOCK>
__device__ void merge_lists(const uint64_t* src, const int* off, const int* cnt, int nl, int kout,
                            uint64_t* out) {
  int total = 0;
  for (int l = 0; l < nl; ++l) total += cnt[l];
  for (int f = threadIdx.x; f < total; f += BLOCK) {
    int l = 0, base = 0;
    while (f >= base + cnt[l]) {
      base += cnt[l];
      ++l;
    }
    const int p = f - base;
    const uint64_t v = src[off[l] + p];
    int rank = p;
    for (int o = 0; o < nl; ++o)
      if (o != l) rank += count_greater(src + off[o], cnt[o], v);
    if (rank < kout) out[rank] = v;
  }
}

// ---------------------------------------------------------------------------------------
// Block-level helpers
// ---------------------------------------------------------------------------------------
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
__device__ T block_scan_excl(T v, T* scratch, T* total) {
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

// Inclusive prefix sum of arr[0, n) in place (n <= BLOCK * 8).
template <int BLOCK>
__device__ void block_scan_array(double* arr, int n, double* scratch) {
  constexpr int ITEMS = 8;
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

// Ascending bitonic sort of arr[0, n) in LDS, n <= cap (cap a power of two).
template <int BLOCK>
__device__ void block_sort_asc(uint64_t* arr, int n, int cap) {
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
        const uint64_t a = arr[lo], b = arr[hi];
        if ((a > b) == asc) {
          arr[lo] = b;
          arr[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  (void)cap;
}

// ---------------------------------------------------------------------------------------
// Candidate finalisation: sorted candidates -> top-p -> min-p -> id-order CDF draw (fp64)
// ---------------------------------------------------------------------------------------
struct FinalShared {
  uint64_t* sorted;  // [kFinalCap] candidates, best first
  double* e;         // [kFinalCap] exp(z - zmax)
  double* cum;       // [kFinalCap] prefix of e (rank order), later id order
  uint64_t* byid;    // [kFinalCap] (id << 32 | rank) for the id-order pass
};

template <int BLOCK>
__device__ void finalize_candidates(const Args& a, int row, int n, FinalShared sh, double* red,
                                    int* s_int) {
  const int t = threadIdx.x;
  const double zmax = (double)composite_z(sh.sorted[0]);
  for (int i = t; i < n; i += BLOCK) {
    const double e = exp((double)composite_z(sh.sorted[i]) - zmax);
    sh.e[i] = e;
    sh.cum[i] = e;
  }
  if (t == 0) {
    s_int[0] = n;  // top-p survivors
    s_int[1] = n;  // min-p survivors
  }
  __syncthreads();
  block_scan_array<BLOCK>(sh.cum, n, red);
  if (a.top_p < 1.0f) {
    const double target = (double)a.top_p * sh.cum[n - 1];
    for (int i = t; i < n; i += BLOCK)
      if (sh.cum[i] >= target && (i == 0 || sh.cum[i - 1] < target)) s_int[0] = i + 1;
  }
  __syncthreads();
  const int lp = s_int[0];
  if (a.min_p > 0.0f) {
    const double mp = (double)a.min_p;
    for (int i = t; i < lp; i += BLOCK)
      if (sh.e[i] < mp && (i == 0 || sh.e[i - 1] >= mp)) s_int[1] = i;
  } else if (t == 0) {
    s_int[1] = lp;
  }
  __syncthreads();
  const int L = s_int[1] < lp ? s_int[1] : lp;
  // kept set = ranks [0, L); order it by id
  for (int i = t; i < L; i += BLOCK)
    sh.byid[i] = ((uint64_t)(uint32_t)composite_id(sh.sorted[i]) << 32) | (uint32_t)i;
  __syncthreads();
  block_sort_asc<BLOCK>(sh.byid, L, kFinalCap);
  for (int i = t; i < L; i += BLOCK) sh.cum[i] = sh.e[(uint32_t)sh.byid[i]];
  __syncthreads();
  block_scan_array<BLOCK>(sh.cum, L, red);
  const double E = sh.cum[L - 1];
  const double target = (double)a.uniforms[row] * E;
  if (t == 0) s_int[2] = L - 1;  // no C_j > u through rounding: last kept id
  __syncthreads();
  for (int i = t; i < L; i += BLOCK)
    if (sh.cum[i] > target && (i == 0 || !(sh.cum[i - 1] > target))) s_int[2] = i;
  __syncthreads();
  if (t == 0) a.out_ids[row] = (int32_t)(sh.byid[s_int[2]] >> 32);
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = t; i < L; i += BLOCK) {
      const uint32_t r = (uint32_t)sh.byid[i];
      prow[sh.byid[i] >> 32] = (float)(sh.e[r] / E);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Row solver
// ---------------------------------------------------------------------------------------
struct SolverShared {
  uint64_t hist_w[256];
  uint32_t hist_c[256];
  uint64_t red64[kSolverBlock / kWave];
  uint32_t red32[kSolverBlock / kWave];
  uint64_t b64[4];
  int32_t b32[8];
};

// exp(z - m) in fp32 with the rounding error of the subtraction folded back (TwoSum).
__device__ __forceinline__ float rel_exp(float z, float m) {
  const float d = z - m;
  const float bb = d - z;
  const float err = (z - (d - bb)) + (-m - bb);
  const float e = expf(d);
  return fmaf(e, err, e);
}
__device__ __forceinline__ uint64_t mass_fixed(float e) {
  return (uint64_t)((double)e * (double)kMassScale);
}

struct CutResult {
  uint64_t cut;   // kept iff composite >= cut
  uint64_t mass;  // fixed-point mass of the kept set
};

// Radix select on the 64-bit rank key over z[0, V): the first element (in rank order)
// at which the running weight reaches `target` (weight 1 if !by_mass, else fixed-point
// mass). If frac > 0 the target is ceil(frac * total weight) of the first round.
template <int BLOCK>
__device__ CutResult radix_cut(const float* z, int V, float zmax, bool by_mass, uint64_t target,
                               double frac, uint32_t key_hi, uint32_t key_lo, SolverShared& sh) {
  const int t = threadIdx.x;
  const uint64_t chi = (uint64_t)key_hi << 32 | 0xFFFFFFFFull;
  const uint64_t clo = (uint64_t)key_lo << 32;
  const int hb = 63 - __clzll(chi ^ clo);
  int shift = (hb >> 3) << 3;
  uint64_t pmask = shift + 8 >= 64 ? 0ull : (~0ull << (shift + 8));
  uint64_t prefix = chi & pmask;
  uint64_t above_mass = 0;
  bool first = true;
  for (;;) {
    if (t < 256) {
      sh.hist_w[t] = 0ull;
      sh.hist_c[t] = 0u;
    }
    __syncthreads();
    for (int i = t; i < V; i += BLOCK) {
      const float v = z[i];
      if (v == -INFINITY) continue;
      const uint64_t c = composite(v, i);
      if ((c & pmask) != prefix) continue;
      const uint32_t d = (uint32_t)(c >> shift) & 255u;
      atomicAdd(&sh.hist_c[d], 1u);
      if (by_mass) {
        atomicAdd((unsigned long long*)&sh.hist_w[d], (unsigned long long)mass_fixed(rel_exp(v, zmax)));
      }
    }
    __syncthreads();
    // bins in descending digit order: thread t <-> digit 255 - t
    uint64_t w = 0;
    uint32_t c = 0;
    if (t < 256) {
      c = sh.hist_c[255 - t];
      w = by_mass ? sh.hist_w[255 - t] : (uint64_t)c;
    }
    uint64_t tot;
    const uint64_t ex = block_scan_excl<BLOCK, uint64_t>(w, sh.red64, &tot);
    if (first && frac > 0.0) {
      const double tg = ceil(frac * (double)tot);
      target = tg < 1.0 ? 1ull : (uint64_t)tg;
      if (target > tot) target = tot;
    }
    first = false;
    if (t == 0) sh.b32[0] = -1;
    __syncthreads();
    if (t < 256 && w > 0 && ex < target && ex + w >= target) {
      sh.b32[0] = 255 - t;
      sh.b64[0] = ex;
      sh.b64[1] = w;
      sh.b32[1] = (int32_t)c;
    }
    __syncthreads();
    const int dsel = sh.b32[0];
    const uint64_t ab = sh.b64[0], wsel = sh.b64[1];
    const uint32_t csel = (uint32_t)sh.b32[1];
    __syncthreads();
    if (dsel < 0) {  // target beyond total weight (all weights zero): keep everything
      CutResult r;
      r.cut = 0ull;
      r.mass = above_mass;
      return r;
    }
    target -= ab;
    // mass of bins strictly above the selected one
    if (by_mass) above_mass += ab;
    prefix |= (uint64_t)dsel << shift;
    pmask |= 255ull << shift;
    const bool done = by_mass ? (csel == 1u) : (target == (uint64_t)csel);
    if (done || shift == 0) {
      CutResult r;
      r.cut = prefix;
      r.mass = above_mass + (by_mass ? wsel : 0ull);
      return r;
    }
    shift -= 8;
  }
}

// The full contract for one row, by one workgroup of BLOCK threads. htab has
// 1 << a.hash_bits slots of LDS.
template <int BLOCK, int DT>
__device__ void solve_row(const Args& a, int row, uint32_t* htab, SolverShared& sh) {
  const int t = threadIdx.x;
  const int V = a.V;
  float* z = a.zbuf + (size_t)row * (size_t)V;
  const void* xrow = row_ptr(a, DT == ARBOR_DTYPE_BF16 ? 2 : 4, row);
  const uint32_t* mrow = a.mask ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const int P = 1 << a.hash_bits;

  // 1. history table of the whole row
  uint32_t flags = 0;
  if (a.H > 0) {
    for (int i = t; i < P; i += BLOCK) htab[i] = kEmptySlot;
    __syncthreads();
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    for (int j = t; j < a.H; j += BLOCK) {
      const int32_t id = h[j];
      if (id < 0) continue;
      if (id >= V)
        flags |= kFlagBadHistory;
      else
        hist_insert(htab, (uint32_t)a.hash_bits, (uint32_t)id);
    }
  }
  // 2. tempered, masked logits
  for (int i = t; i < V; i += BLOCK) {
    float v = Elem<DT>::one(xrow, i) * a.inv_t + 0.0f;
    if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) v = -INFINITY;
    z[i] = v;
  }
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
  uint32_t kmax = 0, kmin = 0xFFFFFFFFu, nf = 0;
  for (int i = t; i < V; i += BLOCK) {
    const float v = z[i];
    if (is_invalid(v)) flags |= kFlagInvalid;
    if (v != -INFINITY && !is_invalid(v)) {
      const uint32_t k = order_key(v);
      kmax = k > kmax ? k : kmax;
      kmin = k < kmin ? k : kmin;
      ++nf;
    }
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

  // 5. cuts: top-k (count), then top-p (mass of the top-k survivors)
  uint64_t cut = 0ull;
  if (a.top_k > 0 && (uint32_t)a.top_k < nf) {
    const CutResult ck = radix_cut<BLOCK>(z, V, zmax, false, (uint64_t)a.top_k, 0.0, kmax, kmin, sh);
    cut = ck.cut;
  }
  if (a.top_p < 1.0f) {
    CutResult cp;
    if (cut != 0ull) {
      // mass of the top-k survivors
      uint64_t m = 0;
      for (int i = t; i < V; i += BLOCK) {
        const float v = z[i];
        if (v != -INFINITY && composite(v, i) >= cut) m += mass_fixed(rel_exp(v, zmax));
      }
      m = block_reduce_sum<BLOCK, uint64_t>(m, sh.red64);
      const double tg = ceil((double)a.top_p * (double)m);
      uint64_t target = tg < 1.0 ? 1ull : (uint64_t)tg;
      if (target > m) target = m;
      cp = radix_cut<BLOCK>(z, V, zmax, true, target, 0.0, kmax, kmin, sh);
    } else {
      cp = radix_cut<BLOCK>(z, V, zmax, true, 0ull, (double)a.top_p, kmax, kmin, sh);
    }
    if (cp.cut > cut) cut = cp.cut;
  }
  const bool use_min_p = a.min_p > 0.0f;

  // 6. kept mass and last kept id
  uint64_t E = 0;
  int32_t last = -1;
  for (int i = t; i < V; i += BLOCK) {
    const float v = z[i];
    if (v == -INFINITY || composite(v, i) < cut) continue;
    const float e = rel_exp(v, zmax);
    if (use_min_p && !(e >= a.min_p)) continue;
    E += mass_fixed(e);
    last = i;
  }
  E = block_reduce_sum<BLOCK, uint64_t>(E, sh.red64);
  last = block_reduce_max<BLOCK, int32_t>(last, (int32_t*)sh.red32);

  // 7. draw: first id (ascending) whose running mass exceeds floor(u * E)
  const double uE = (double)a.uniforms[row] * (double)E;
  uint64_t target;
  if (uE >= 0.0)
    target = uE >= 18446744073709549568.0 ? ~0ull : (uint64_t)uE;
  else
    target = uE < 0.0 ? 0ull : ~0ull;  // NaN: no crossing
  const double Ed = (double)E / (double)kMassScale;
  if (t == 0) sh.b32[2] = -1;
  __syncthreads();
  uint64_t running = 0;
  constexpr int IT = 4;
  for (int base = 0; base < V; base += BLOCK * IT) {
    uint64_t w[IT];
    uint64_t loc = 0;
#pragma unroll
    for (int j = 0; j < IT; ++j) {
      const int i = base + t * IT + j;
      w[j] = 0;
      float q = 0.0f;
      if (i < V) {
        const float v = z[i];
        if (v != -INFINITY && composite(v, i) >= cut) {
          const float e = rel_exp(v, zmax);
          if (!use_min_p || e >= a.min_p) {
            w[j] = mass_fixed(e);
            q = (float)((double)e / Ed);
          }
        }
        if (prow) prow[i] = q;
      }
      loc += w[j];
    }
    uint64_t tot;
    const uint64_t ex = block_scan_excl<BLOCK, uint64_t>(loc, sh.red64, &tot);
    const uint64_t b0 = running + ex;
    if (b0 <= target && b0 + loc > target) {
      uint64_t acc = b0;
#pragma unroll
      for (int j = 0; j < IT; ++j) {
        acc += w[j];
        if (acc > target) {
          sh.b32[2] = base + t * IT + j;
          break;
        }
      }
    }
    running += tot;
    __syncthreads();
    if (sh.b32[2] >= 0 && !prow) break;
  }
  if (t == 0) a.out_ids[row] = sh.b32[2] >= 0 ? sh.b32[2] : last;
}

// ---------------------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(kSolverBlock) solver_kernel(Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SolverShared sh;
  solve_row<kSolverBlock, DT>(a, blockIdx.x, reinterpret_cast<uint32_t*>(smem), sh);
}

// Dynamic LDS of stream_kernel, in bytes, for a given history table / chunk bitmap.
__host__ __device__ constexpr size_t stream_lds_bytes(int hash_slots, int bitmap_words) {
  return sizeof(uint64_t) * kStreamWaves * kWaveCap + sizeof(uint32_t) * kStreamWaves * 256 +
         sizeof(uint32_t) * (size_t)(hash_slots + bitmap_words);
}

template <int DT, bool PEN, bool MASK, bool MODE_K>
__global__ void __launch_bounds__(kStreamBlock) stream_kernel(Args a) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int ESZ = DT == ARBOR_DTYPE_BF16 ? 2 : 4;
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* wbuf = reinterpret_cast<uint64_t*>(smem);
  uint32_t* whist = reinterpret_cast<uint32_t*>(wbuf + kStreamWaves * kWaveCap);
  uint32_t* htab = whist + kStreamWaves * 256;
  uint32_t* bitmap = htab + (PEN ? (1 << a.hash_bits) : 0);
  __shared__ uint32_t s_flags;
  __shared__ int s_cnt[kMaxChunks];
  __shared__ int s_off[kMaxChunks];
  __shared__ int s_last;
  __shared__ int s_int[4];
  __shared__ double s_red[kStreamWaves];

  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  int row, chunk;
  if (a.xcd_map) {
    const int g = blockIdx.x, xcd = g & 7, slot = g >> 3;
    row = (slot / a.S) * 8 + xcd;
    chunk = slot % a.S;
  } else {
    row = blockIdx.x / a.S;
    chunk = blockIdx.x % a.S;
  }
  if (row >= a.B) return;
  const int c0 = chunk * a.chunk_len;
  const int c1 = min(a.V, c0 + a.chunk_len);
  const void* xrow = row_ptr(a, ESZ, row);

  if (t == 0) s_flags = 0u;
  if (PEN) {
    const int P = 1 << a.hash_bits;
    for (int i = t; i < P; i += kStreamBlock) htab[i] = kEmptySlot;
    for (int i = t; i < a.bitmap_words; i += kStreamBlock) bitmap[i] = 0u;
    __syncthreads();
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    bool bad = false;
    for (int j = t; j < a.H; j += kStreamBlock) {
      const int32_t id = h[j];
      if (id >= a.V) {
        bad = true;
      } else if (id >= c0 && id < c1) {
        hist_insert(htab, (uint32_t)a.hash_bits, (uint32_t)id);
        atomicOr(&bitmap[(id - c0) >> 5], 1u << ((id - c0) & 31));
      }
    }
    if (bad) atomicOr(&s_flags, kFlagBadHistory);
  }
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = c0 + t; i < c1; i += kStreamBlock) prow[i] = 0.0f;
  }
  __syncthreads();

  // ---- stream the chunk ----
  uint64_t* buf = wbuf + wave * kWaveCap;
  uint32_t* rh = whist + wave * 256;
  int wc = 0;
  float thr = -INFINITY;
  bool bad = false, ovf = false;
  const uint32_t* mrow = MASK ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const bool aligned = a.aligned != 0;
  const int n_units = (c1 - c0 + VEC - 1) / VEC;
  for (int ub = wave * kUnroll * kWave; ub < n_units && !ovf; ub += kStreamWaves * kUnroll * kWave) {
    float x[kUnroll][VEC];
    uint32_t mw[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int e0 = c0 + (ub + u * kWave + lane) * VEC;
      load_unit<DT>(xrow, e0, c1, aligned, x[u]);
      if (MASK) mw[u] = e0 < c1 ? mrow[e0 >> 5] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int e0 = c0 + (ub + u * kWave + lane) * VEC;
      float z[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) z[j] = x[u][j] * a.inv_t;
      if (PEN && e0 < c1) {
        const uint32_t bits = (bitmap[(e0 - c0) >> 5] >> ((e0 - c0) & 31)) & ((1u << VEC) - 1u);
        if (bits) {
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            if ((bits >> j) & 1u)
              z[j] = penalize(z[j], hist_count(htab, (uint32_t)a.hash_bits, (uint32_t)(e0 + j)), a.pen);
        }
      }
      if (MASK) {
        const uint32_t m = mw[u] >> (e0 & 31);
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          if (!((m >> j) & 1u)) z[j] = -INFINITY;
      }
      bool any = false;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        bad |= is_invalid(z[j]);
        any |= z[j] > thr && !is_invalid(z[j]);
      }
      if (__ballot(any)) {
        if (wc > kWaveCap - kWave * VEC) {
          if (MODE_K)
            thr = wave_keep_topk(buf, wc, a.top_k, rh);
          else
            thr = wave_keep_band(buf, wc, a.ln_min_p_lo);
          if (wc > kWaveCap - kWave * VEC) {
            ovf = true;
            break;
          }
        }
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const bool take = z[j] > thr && !is_invalid(z[j]);
          const uint64_t bal = __ballot(take);
          if (bal) {
            if (take) buf[wc + lanes_below(bal)] = composite(z[j] + 0.0f, e0 + j);
            wc += __popcll(bal);
          }
        }
      }
    }
  }
  // final per-wave list: top-k (or min-p band), sorted best first
  if (!ovf) {
    if (MODE_K) {
      if (wc > a.top_k) wave_keep_topk(buf, wc, a.top_k, rh);
    } else if (wc > 0) {
      wave_keep_band(buf, wc, a.ln_min_p_lo);
    }
    if (wc > kChunkSlot)
      ovf = true;
    else
      wave_sort_desc(buf, wc);
  }
  if (__ballot(bad) && lane == 0) atomicOr(&s_flags, kFlagInvalid);
  if (ovf && lane == 0) atomicOr(&s_flags, kFlagOverflow);
  if (lane == 0) {
    s_cnt[wave] = ovf ? 0 : wc;
    s_off[wave] = wave * kWaveCap;
  }
  __syncthreads();

  // ---- chunk list: merge the wave lists, publish ----
  const size_t slot_base = ((size_t)row * (size_t)a.S + (size_t)chunk);
  uint64_t* gl = a.cand + slot_base * kChunkSlot;
  uint32_t flags = s_flags;
  int kout;
  if (MODE_K) {
    int tot = 0;
    for (int w = 0; w < kStreamWaves; ++w) tot += s_cnt[w];
    kout = min(a.top_k, tot);
  } else {
    // drop what falls outside the band of the chunk's best z
    float best = -INFINITY;
    for (int w = 0; w < kStreamWaves; ++w)
      if (s_cnt[w] > 0) best = fmaxf(best, composite_z(wbuf[w * kWaveCap]));
    const float thr_c = best + a.ln_min_p_lo;
    __syncthreads();
    if (t < kStreamWaves && s_cnt[t] > 0) {
      const uint64_t* L = wbuf + t * kWaveCap;
      int lo = 0, hi = s_cnt[t];
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (composite_z(L[mid]) >= thr_c)
          lo = mid + 1;
        else
          hi = mid;
      }
      s_cnt[t] = lo;
    }
    __syncthreads();
    int tot = 0;
    for (int w = 0; w < kStreamWaves; ++w) tot += s_cnt[w];
    if (tot > a.chunk_cap) {
      flags |= kFlagOverflow;
      tot = 0;
    }
    kout = tot;
  }
  if (!(flags & kFlagOverflow)) merge_lists<kStreamBlock>(wbuf, s_off, s_cnt, kStreamWaves, kout, gl);
  if (t == 0) {
    a.hdr[slot_base * 4 + 0] = (uint32_t)((flags & kFlagOverflow) ? 0 : kout);
    a.hdr[slot_base * 4 + 1] = flags;
  }

  // ---- arrival: the last chunk of the row finishes it ----
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const uint32_t prev = atomicAdd(&a.counters[row], 1u);
    s_last = prev == (uint32_t)(a.S - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (t == 0) a.counters[row] = 0u;

  uint32_t rflags = 0;
  for (int c = 0; c < a.S; ++c) rflags |= a.hdr[((size_t)row * a.S + c) * 4 + 1];
  if (rflags & kFlagBadHistory) {
    if (t == 0) a.out_ids[row] = ARBOR_ID_BAD_HISTORY;
    return;
  }
  if (rflags & kFlagInvalid) {
    if (t == 0) a.out_ids[row] = ARBOR_ID_INVALID;
    return;
  }
  if (rflags & kFlagOverflow) {
    SolverShared& ssh = *reinterpret_cast<SolverShared*>(wbuf);
    __syncthreads();
    solve_row<kStreamBlock, DT>(a, row, htab, ssh);
    return;
  }
  // gather the S chunk lists into LDS
  uint64_t* lists = wbuf;                       // [kFinalCap]
  uint64_t* sorted = wbuf + kFinalCap;          // [kFinalCap]
  double* e = reinterpret_cast<double*>(wbuf + 2 * kFinalCap);
  double* cum = reinterpret_cast<double*>(wbuf + 3 * kFinalCap);
  __syncthreads();
  if (t == 0) {
    int off = 0;
    for (int c = 0; c < a.S; ++c) {
      const int n = (int)a.hdr[((size_t)row * a.S + c) * 4 + 0];
      s_cnt[c] = n;
      s_off[c] = off;
      off += n;
    }
    s_int[3] = off;
  }
  __syncthreads();
  const int total = s_int[3];
  if (total == 0) {
    if (t == 0) a.out_ids[row] = ARBOR_ID_EMPTY;
    return;
  }
  for (int c = 0; c < a.S; ++c) {
    const uint64_t* src = a.cand + ((size_t)row * a.S + c) * kChunkSlot;
    for (int i = t; i < s_cnt[c]; i += kStreamBlock) lists[s_off[c] + i] = src[i];
  }
  __syncthreads();
  int n;
  if (MODE_K) {
    n = min(a.top_k, total);
  } else {
    // band of the row's best z
    if (t == 0) {
      float best = -INFINITY;
      for (int c = 0; c < a.S; ++c)
        if (s_cnt[c] > 0) best = fmaxf(best, composite_z(lists[s_off[c]]));
      const float thr_r = best + a.ln_min_p_lo;
      int tot = 0;
      for (int c = 0; c < a.S; ++c) {
        const uint64_t* L = lists + s_off[c];
        int lo = 0, hi = s_cnt[c];
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (composite_z(L[mid]) >= thr_r)
            lo = mid + 1;
          else
            hi = mid;
        }
        s_cnt[c] = lo;
        tot += lo;
      }
      s_int[3] = tot;
    }
    __syncthreads();
    n = s_int[3];
  }
  merge_lists<kStreamBlock>(lists, s_off, s_cnt, a.S, n, sorted);
  __syncthreads();
  FinalShared fs;
  fs.sorted = sorted;
  fs.e = e;
  fs.cum = cum;
  fs.byid = lists;
  finalize_candidates<kStreamBlock>(a, row, n, fs, s_red, s_int);
}

}  // namespace arbor

// =======================================================================================
// Host side: validation, path selection, launch, C ABI
// =======================================================================================
namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  snprintf(g_err, sizeof g_err, "%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
  return (int)e;
}

enum class Path { Stream, Solver };

struct Plan {
  Path path;
  bool mode_k;
  int k;            // effective top-k (0 = off)
  int S, chunk_len, chunk_cap;
  int hash_bits, bitmap_words;
  size_t lds;
  // workspace layout (byte offsets)
  size_t off_counters, off_hdr, off_cand, off_zbuf, total;
};

int validate(const arbor_sampling_params* p) {
  if (!p) return fail(ARBOR_ERR_NULL, "params is NULL");
  if (p->struct_size != sizeof(arbor_sampling_params))
    return fail(ARBOR_ERR_STRUCT_SIZE, "params->struct_size is %u, expected %zu", p->struct_size,
                sizeof(arbor_sampling_params));
  if (p->batch <= 0 || p->vocab <= 0 || p->vocab > ARBOR_VOCAB_MAX || p->ld_logits < p->vocab)
    return fail(ARBOR_ERR_SHAPE, "bad shape: batch %d, vocab %d (max %d), ld_logits %d", p->batch, p->vocab,
                ARBOR_VOCAB_MAX, p->ld_logits);
  if (p->dtype != ARBOR_DTYPE_F32 && p->dtype != ARBOR_DTYPE_BF16)
    return fail(ARBOR_ERR_DTYPE, "unknown dtype %d", p->dtype);
  if (!(p->temperature > 0.0f) || !std::isfinite(p->temperature))
    return fail(ARBOR_ERR_TEMPERATURE, "temperature must be finite and > 0, got %g", (double)p->temperature);
  if (!(p->repetition_penalty > 0.0f) || !std::isfinite(p->repetition_penalty) || !std::isfinite(p->frequency_penalty) ||
      !std::isfinite(p->presence_penalty))
    return fail(ARBOR_ERR_PENALTY, "penalties must be finite (repetition > 0): %g %g %g",
                (double)p->repetition_penalty, (double)p->frequency_penalty, (double)p->presence_penalty);
  if (p->top_k < 0) return fail(ARBOR_ERR_TOP_K, "top_k must be >= 0, got %d", p->top_k);
  if (!(p->top_p > 0.0f && p->top_p <= 1.0f))
    return fail(ARBOR_ERR_TOP_P, "top_p must be in (0, 1], got %g", (double)p->top_p);
  if (!(p->min_p >= 0.0f && p->min_p < 1.0f))
    return fail(ARBOR_ERR_MIN_P, "min_p must be in [0, 1), got %g", (double)p->min_p);
  if (p->hist_len < 0 || p->hist_len > ARBOR_HISTORY_MAX)
    return fail(ARBOR_ERR_HISTORY, "hist_len must be in [0, %d], got %d", ARBOR_HISTORY_MAX, p->hist_len);
  if (p->flags & ~ARBOR_FLAG_WRITE_PROBS) return fail(ARBOR_ERR_FLAGS, "unknown flag bits 0x%x", p->flags);
  return ARBOR_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

Plan make_plan(const arbor_sampling_params* p) {
  Plan pl{};
  const int V = p->vocab, B = p->batch;
  pl.k = (p->top_k > 0 && p->top_k < V) ? p->top_k : 0;
  const bool minp_only = pl.k == 0 && p->top_p >= 1.0f && p->min_p > 0.0f;
  if (pl.k > 0 && pl.k <= arbor::kMaxTopK) {
    pl.path = Path::Stream;
    pl.mode_k = true;
  } else if (minp_only) {
    pl.path = Path::Stream;
    pl.mode_k = false;
  } else {
    pl.path = Path::Solver;
  }
  int hb = 6;
  while ((1 << hb) < 2 * p->hist_len) ++hb;
  pl.hash_bits = hb;
  if (pl.path == Path::Stream) {
    // chunks: enough workgroups to fill the chip, each chunk a multiple of 512 elements
    const int target_wg = 2048;
    int S = (target_wg + B - 1) / B;
    const int max_by_len = (V + 2047) / 2048;  // at least ~2K elements per chunk
    if (S > max_by_len) S = max_by_len;
    const int smax = pl.mode_k ? arbor::kFinalCap / pl.k : arbor::kFinalCap / 16;
    if (S > smax) S = smax;
    if (S > arbor::kMaxChunks) S = arbor::kMaxChunks;
    if (S < 1) S = 1;
    int len = (int)align_up((size_t)((V + S - 1) / S), 512);
    S = (V + len - 1) / len;
    pl.S = S;
    pl.chunk_len = len;
    pl.chunk_cap = arbor::kFinalCap / S < arbor::kChunkSlot ? arbor::kFinalCap / S : arbor::kChunkSlot;
    const bool pen = p->hist_len > 0;
    pl.bitmap_words = pen ? len / 32 : 0;
    pl.lds = arbor::stream_lds_bytes(pen ? (1 << hb) : 0, pl.bitmap_words);
  } else {
    pl.S = 0;
    pl.lds = sizeof(uint32_t) * (size_t)(1 << hb);
  }
  size_t off = 0;
  pl.off_counters = off;
  off = align_up(off + sizeof(uint32_t) * (size_t)B, 256);
  pl.off_hdr = off;
  off = align_up(off + sizeof(uint32_t) * 4 * (size_t)B * (size_t)pl.S, 256);
  pl.off_cand = off;
  off = align_up(off + sizeof(uint64_t) * arbor::kChunkSlot * (size_t)B * (size_t)pl.S, 256);
  pl.off_zbuf = off;
  off = align_up(off + sizeof(float) * (size_t)B * (size_t)V, 256);
  pl.total = off;
  return pl;
}

template <typename K>
int launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, const arbor::Args& a) {
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute");
  }
  hipLaunchKernelGGL(kernel, grid, block, lds, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return ARBOR_OK;
}

template <int DT, bool PEN, bool MASK>
int launch_stream(bool mode_k, dim3 grid, size_t lds, hipStream_t st, const arbor::Args& a) {
  const dim3 block(arbor::kStreamBlock);
  if (mode_k) return launch(arbor::stream_kernel<DT, PEN, MASK, true>, grid, block, lds, st, a);
  return launch(arbor::stream_kernel<DT, PEN, MASK, false>, grid, block, lds, st, a);
}

template <int DT>
int launch_stream_dt(bool pen, bool mask, bool mode_k, dim3 grid, size_t lds, hipStream_t st,
                     const arbor::Args& a) {
  if (pen) {
    if (mask) return launch_stream<DT, true, true>(mode_k, grid, lds, st, a);
    return launch_stream<DT, true, false>(mode_k, grid, lds, st, a);
  }
  if (mask) return launch_stream<DT, false, true>(mode_k, grid, lds, st, a);
  return launch_stream<DT, false, false>(mode_k, grid, lds, st, a);
}

}  // namespace

extern "C" {

int arbor_abi_version(void) { return ARBOR_ABI_VERSION; }

const char* arbor_last_error(void) { return g_err; }

void arbor_sampling_params_init(arbor_sampling_params* p, int32_t batch, int32_t vocab) {
  if (!p) return;
  memset(p, 0, sizeof *p);
  p->struct_size = sizeof(arbor_sampling_params);
  p->batch = batch;
  p->vocab = vocab;
  p->ld_logits = vocab;
  p->dtype = ARBOR_DTYPE_F32;
  p->temperature = 1.0f;
  p->repetition_penalty = 1.0f;
  p->top_p = 1.0f;
  p->mask_words = (vocab + 31) / 32;
}

size_t arbor_sample_workspace_bytes(const arbor_sampling_params* p) {
  if (validate(p) != ARBOR_OK) return 0;
  return make_plan(p).total;
}

int arbor_sample(const arbor_sampling_params* p, const void* logits, const int32_t* history,
                 const uint32_t* allow_mask, const float* uniforms, int32_t* out_ids, float* out_probs,
                 void* workspace, size_t workspace_bytes, void* stream) {
  int st = validate(p);
  if (st != ARBOR_OK) return st;
  if (!logits || !uniforms || !out_ids) return fail(ARBOR_ERR_NULL, "logits, uniforms and out_ids are required");
  if (p->hist_len > 0 && !history) return fail(ARBOR_ERR_HISTORY, "history is NULL with hist_len %d", p->hist_len);
  if (allow_mask && p->mask_words < (p->vocab + 31) / 32)
    return fail(ARBOR_ERR_MASK, "mask_words %d < ceil(vocab / 32) = %d", p->mask_words, (p->vocab + 31) / 32);
  const bool probs = (p->flags & ARBOR_FLAG_WRITE_PROBS) != 0;
  if (probs && !out_probs) return fail(ARBOR_ERR_FLAGS, "ARBOR_FLAG_WRITE_PROBS without out_probs");
  const Plan pl = make_plan(p);
  if (!workspace || workspace_bytes < pl.total)
    return fail(ARBOR_ERR_WORKSPACE, "workspace of %zu bytes given, %zu needed", workspace ? workspace_bytes : 0,
                pl.total);

  arbor::Args a{};
  a.logits = logits;
  a.ld = p->ld_logits;
  a.V = p->vocab;
  a.B = p->batch;
  a.hist = history;
  a.H = p->hist_len;
  a.mask = allow_mask;
  a.mask_words = p->mask_words;
  a.uniforms = uniforms;
  a.out_ids = out_ids;
  a.out_probs = out_probs;
  a.inv_t = 1.0f / p->temperature;
  a.pen.rp = p->repetition_penalty;
  a.pen.inv_rp = 1.0f / p->repetition_penalty;
  a.pen.fp = p->frequency_penalty;
  a.pen.pp = p->presence_penalty;
  a.top_k = pl.k;
  a.top_p = p->top_p;
  a.min_p = p->min_p;
  a.ln_min_p_lo = p->min_p > 0.0f ? (float)(log((double)p->min_p) - 1e-3) : -INFINITY;
  a.S = pl.S;
  a.chunk_len = pl.chunk_len;
  a.chunk_cap = pl.chunk_cap;
  a.hash_bits = pl.hash_bits;
  a.bitmap_words = pl.bitmap_words;
  const size_t esz = p->dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
  a.aligned = ((uintptr_t)logits % 16 == 0) && (((size_t)p->ld_logits * esz) % 16 == 0);
  a.write_probs = probs ? 1 : 0;
  char* ws = static_cast<char*>(workspace);
  a.counters = reinterpret_cast<uint32_t*>(ws + pl.off_counters);
  a.hdr = reinterpret_cast<uint32_t*>(ws + pl.off_hdr);
  a.cand = reinterpret_cast<uint64_t*>(ws + pl.off_cand);
  a.zbuf = reinterpret_cast<float*>(ws + pl.off_zbuf);
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (pl.path == Path::Solver) {
    const dim3 grid(p->batch), block(arbor::kSolverBlock);
    if (p->dtype == ARBOR_DTYPE_BF16) return launch(arbor::solver_kernel<ARBOR_DTYPE_BF16>, grid, block, pl.lds, s, a);
    return launch(arbor::solver_kernel<ARBOR_DTYPE_F32>, grid, block, pl.lds, s, a);
  }
  a.xcd_map = (p->batch % 8 == 0) ? 1 : 0;
  const dim3 grid((unsigned)(p->batch * pl.S));
  const bool pen = p->hist_len > 0, mask = allow_mask != nullptr;
  if (p->dtype == ARBOR_DTYPE_BF16)
    return launch_stream_dt<ARBOR_DTYPE_BF16>(pen, mask, pl.mode_k, grid, pl.lds, s, a);
  return launch_stream_dt<ARBOR_DTYPE_F32>(pen, mask, pl.mode_k, grid, pl.lds, s, a);
}

int arbor_device_count(int* count) {
  if (!count) return fail(ARBOR_ERR_NULL, "count is NULL");
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return fail(ARBOR_ERR_NO_DEVICE, "no HIP device is visible");
  }
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  return ARBOR_OK;
}

int arbor_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(ARBOR_ERR_NULL, "ptr is NULL");
  hipError_t e = hipMalloc(ptr, bytes);
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "hipMalloc");
}

int arbor_free(void* ptr) {
  if (!ptr) return ARBOR_OK;
  hipError_t e = hipFree(ptr);
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "hipFree");
}

int arbor_memcpy(void* dst, const void* src, size_t bytes, int kind) {
  if (kind < 0 || kind > 4) return fail(ARBOR_ERR_FLAGS, "memcpy kind %d not in 0..4", kind);
  if (bytes == 0) return ARBOR_OK;
  if (!dst || !src) return fail(ARBOR_ERR_NULL, "memcpy with a NULL pointer");
  hipError_t e = hipMemcpy(dst, src, bytes, static_cast<hipMemcpyKind>(kind));
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "hipMemcpy");
}

int arbor_memset(void* ptr, int value, size_t bytes) {
  if (bytes == 0) return ARBOR_OK;
  if (!ptr) return fail(ARBOR_ERR_NULL, "memset of a NULL pointer");
  hipError_t e = hipMemset(ptr, value, bytes);
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "hipMemset");
}

int arbor_synchronize(void) {
  hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "hipDeviceSynchronize");
}

}  // extern "C"
