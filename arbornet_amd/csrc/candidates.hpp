// candidates.hpp -- candidate lists of the streaming path and the fp64 finish of a row.
//
// A candidate is a 64-bit rank key (order_key(z) << 32 | ~id): larger = earlier in the
// ranking z descending, id ascending. A wave keeps its candidates in a private LDS
// buffer; lists that leave a wave are sorted best first.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"
#include "row_solver.hpp"

namespace arbor {

// ---------------------------------------------------------------------------------------
// Wave level
// ---------------------------------------------------------------------------------------

// Keep exactly the k best of the n (> k) composites of a wave buffer, unsorted, in
// buf[0, k). Returns the z of the k-th best: a valid acceptance threshold (z >= thr) for
// everything the wave sees afterwards. MSB-first radix select, 8-bit digits taken just
// below the highest bit in which the entries differ.
template <int CAP>
__device__ __forceinline__ float wave_keep_topk(uint64_t* buf, int& n, int k, uint32_t* hist) {
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
  int shift = hb >= 7 ? hb - 7 : 0;
  uint64_t pmask = hb >= 63 ? 0ull : (~0ull << (hb + 1));
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
    if (bal == 0ull) {  // unreachable (need <= number of matching entries); keep everything
      prefix = 0ull;
      break;
    }
    const int src = __ffsll((long long)bal) - 1;
    dsel = lane_get(dsel, src);
    above = lane_get(above, src);
    csel = lane_get(csel, src);
    need -= above;
    prefix = (prefix & ~(255ull << shift)) | ((uint64_t)dsel << shift);
    pmask |= 255ull << shift;
    if (need == csel || shift == 0) break;
    shift = shift >= 8 ? shift - 8 : 0;
  }
  // keep every composite >= prefix: the selected bin and everything above it
  constexpr int R = CAP / kWave;
  uint64_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWave + lane;
    v[r] = i < n ? buf[i] : 0ull;
  }
  wave_lds_sync();
  int nn = 0;
  uint64_t mn = ~0ull;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool keep = v[r] != 0ull && v[r] >= prefix;
    const uint64_t bal = __ballot(keep);
    if (keep) {
      buf[nn + lanes_below(bal)] = v[r];
      mn = v[r] < mn ? v[r] : mn;
    }
    nn += __popcll(bal);
  }
  wave_lds_sync();
  n = uniform<int>(nn);
  mn = wave_min(mn);
  return nn > 0 ? composite_z(mn) : -FLT_MAX;
}

// Keep the entries with z >= (largest z) + band (band < 0). Returns that threshold.
template <int CAP>
__device__ float wave_keep_band(uint64_t* buf, int& n, float band) {
  const int lane = lane_id();
  uint64_t hi = 0;
  for (int i = lane; i < n; i += kWave) {
    const uint64_t c = buf[i];
    hi = c > hi ? c : hi;
  }
  hi = wave_max(hi);
  const float thr = composite_z(hi) + band;
  constexpr int R = CAP / kWave;
  uint64_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWave + lane;
    v[r] = i < n ? buf[i] : 0ull;
  }
  wave_lds_sync();
  int nn = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool keep = v[r] != 0ull && composite_z(v[r]) >= thr;
    const uint64_t bal = __ballot(keep);
    if (keep) buf[nn + lanes_below(bal)] = v[r];
    nn += __popcll(bal);
  }
  wave_lds_sync();
  n = nn;
  return thr;
}

// Sort n <= CAP composites of a wave buffer descending.
template <int CAP>
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
  constexpr int R = CAP / kWave;
  uint64_t v[R];
  int rank[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWave + lane;
    v[r] = i < n ? buf[i] : 0ull;
    rank[r] = 0;
  }
  for (int j = 0; j < n; ++j) {
    const uint64_t c = buf[j];
#pragma unroll
    for (int r = 0; r < R; ++r) rank[r] += c > v[r] ? 1 : 0;
  }
  wave_lds_sync();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r * kWave + lane < n) buf[rank[r]] = v[r];
  wave_lds_sync();
}

// ---------------------------------------------------------------------------------------
// Workgroup level: LDS layout of the streaming / finishing workgroups
// ---------------------------------------------------------------------------------------
struct SolverShared;

// Dynamic LDS: region A = wave buffers (stream) / history table + chunk lists (finish);
// region B = radix histograms + chunk bitmap (stream) / finish arrays (finish).
__host__ __device__ constexpr size_t lds_region_a() { return sizeof(uint64_t) * kWaves * kWaveCap; }
__host__ __device__ constexpr size_t lds_fin_bytes() { return sizeof(uint64_t) * 5 * kFinalCap; }
__host__ __device__ constexpr size_t lds_stream_b(int bitmap_words) {
  return sizeof(uint32_t) * ((size_t)kWaves * 256 + (size_t)bitmap_words);
}
__host__ __device__ constexpr size_t lds_total(int bitmap_words) {
  return lds_region_a() + (lds_stream_b(bitmap_words) > lds_fin_bytes() ? lds_stream_b(bitmap_words) : lds_fin_bytes());
}

struct Lds {
  uint64_t* wbuf;     // [kWaves * kWaveCap]
  uint32_t* htab;     // overlays wbuf[0, 4096): history table (<= 8192 slots)
  uint64_t* lists;    // overlays wbuf[4096, 8192): chunk lists in the finish kernel
  uint32_t* whist;    // [kWaves * 256]
  uint32_t* bitmap;   // [bitmap_words]
  uint64_t* uni;      // [kFinalCap]  candidate union
  uint64_t* sorted;   // [kFinalCap]
  double* e;          // [kFinalCap]
  double* cum;        // [kFinalCap]
  uint64_t* byid;     // [kFinalCap]
  SolverShared* ssh;  // overlays region B (row-solver fallback)

  __device__ explicit Lds(unsigned char* base) {
    wbuf = reinterpret_cast<uint64_t*>(base);
    htab = reinterpret_cast<uint32_t*>(base);
    lists = wbuf + kWaves * kWaveCap / 2;
    unsigned char* b = base + lds_region_a();
    whist = reinterpret_cast<uint32_t*>(b);
    bitmap = whist + kWaves * 256;
    uni = reinterpret_cast<uint64_t*>(b);
    sorted = uni + kFinalCap;
    e = reinterpret_cast<double*>(sorted + kFinalCap);
    cum = e + kFinalCap;
    byid = reinterpret_cast<uint64_t*>(cum + kFinalCap);
    ssh = reinterpret_cast<SolverShared*>(b);
  }
};

struct FinishShared {
  uint64_t t0;       // top-k lower bound (composite)
  float zthr;        // min-p band threshold (z)
  int n_uni;
  int uni_over;
  uint32_t flags;
  int cnt[kMaxChunks > kWaves ? kMaxChunks : kWaves];
  int off[kMaxChunks > kWaves ? kMaxChunks : kWaves];
  int pc[kMaxChunks > kWaves ? kMaxChunks : kWaves];
  int po[kMaxChunks > kWaves ? kMaxChunks : kWaves];
  double red[kWaves];
  int ints[4];
  int next_batch;  // streaming: next batch index to hand out
};

// Union of the prefixes of nl sorted lists that can still reach the final selection:
// top-k: entries >= t0, t0 = k-th best of the first h entries of every list (the k-th
// best of a subset bounds the k-th best of the whole row from below); min-p: entries
// with z >= (best head) + band. Writes s.uni / s.n_uni / s.uni_over.
template <int BLOCK, bool MODE_K>
__device__ void gather_prefixes(const Args& a, const uint64_t* lists, int nl, Lds& L, FinishShared& s) {
  const int t = threadIdx.x;
  if (t < kWave) {
    if (MODE_K) {
      const int h = kWave / nl > 0 ? kWave / nl : 1;
      const int l = t / h, pos = t % h;
      uint64_t v = (l < nl && pos < s.cnt[l]) ? lists[s.off[l] + pos] : 0ull;
      v = wave_sort64_desc(v);
      const uint64_t kth = lane_get(v, a.top_k - 1);
      if (t == 0) s.t0 = kth;
    } else {
      float m = -INFINITY;
      for (int l = t; l < nl; l += kWave)
        if (s.cnt[l] > 0) m = fmaxf(m, composite_z(lists[s.off[l]]));
      m = wave_max(m);
      if (t == 0) s.zthr = m + a.ln_min_p_lo;
    }
  }
  __syncthreads();
  if (t < nl) {
    const uint64_t* Lp = lists + s.off[t];
    int lo = 0, hi = s.cnt[t];
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const bool keep = MODE_K ? (Lp[mid] >= s.t0) : (composite_z(Lp[mid]) >= s.zthr);
      if (keep)
        lo = mid + 1;
      else
        hi = mid;
    }
    s.pc[t] = lo;
  }
  __syncthreads();
  if (t == 0) {
    int o = 0;
    for (int l = 0; l < nl; ++l) {
      s.po[l] = o;
      o += s.pc[l];
    }
    s.uni_over = o > kFinalCap ? 1 : 0;
    s.n_uni = o > kFinalCap ? kFinalCap : o;
  }
  __syncthreads();
  for (int l = 0; l < nl; ++l) {
    const int base = s.po[l], n = s.pc[l];
    for (int i = t; i < n && base + i < kFinalCap; i += BLOCK) L.uni[base + i] = lists[s.off[l] + i];
  }
  __syncthreads();
}

// Penalised logits of the row's distinct history ids, added to the union (they were
// excluded from the stream). Also flags history ids >= vocab and NaN / +inf results.
template <int BLOCK, int DT, bool MODE_K>
__device__ void history_candidates(const Args& a, int row, Lds& L, FinishShared& s) {
  const int t = threadIdx.x;
  const int P = 1 << a.hash_bits;
  for (int i = t; i < P; i += BLOCK) L.htab[i] = kEmptySlot;
  __syncthreads();
  constexpr int R = (ARBOR_HISTORY_MAX + BLOCK - 1) / BLOCK;
  const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = a.mask ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  int own[R];
  float xo[R];
  uint32_t mo[R];
  bool bad = false, inv = false;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int j = t + r * BLOCK;
    own[r] = -1;
    if (j < a.H) {
      const int32_t id = h[j];
      if (id >= a.V)
        bad = true;
      else if (id >= 0 && hist_insert(L.htab, (uint32_t)a.hash_bits, (uint32_t)id))
        own[r] = id;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    xo[r] = 0.0f;
    mo[r] = ~0u;
    if (own[r] >= 0) {
      xo[r] = Elem<DT>::one(xrow, own[r]);
      if (mrow) mo[r] = mrow[own[r] >> 5];
    }
  }
  __syncthreads();  // every occurrence counted
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (own[r] < 0) continue;
    const int32_t id = own[r];
    float z = penalize(xo[r] * a.inv_t + 0.0f, hist_count(L.htab, (uint32_t)a.hash_bits, (uint32_t)id), a.pen);
    if (!((mo[r] >> (id & 31)) & 1u)) z = -INFINITY;
    if (is_invalid(z)) {
      inv = true;
    } else if (z != -INFINITY) {
      const uint64_t c = composite(z, id);
      // below the non-history bound the final cut can only be higher: drop it here
      if (MODE_K ? c >= s.t0 : z >= s.zthr) {
        const int pos = atomicAdd(&s.n_uni, 1);
        if (pos < kFinalCap)
          L.uni[pos] = c;
        else
          s.uni_over = 1;
      }
    }
  }
  if (bad) atomicOr(&s.flags, kFlagBadHistory);
  if (inv) atomicOr(&s.flags, kFlagInvalid);
  __syncthreads();
  if (t == 0 && s.n_uni > kFinalCap) s.n_uni = kFinalCap;
  __syncthreads();
}

// sorted[0, n) best first -> top-p -> min-p -> id-order CDF draw, all in fp64.
template <int BLOCK>
__device__ void finalize_candidates(const Args& a, int row, int n, Lds& L, FinishShared& s) {
  const int t = threadIdx.x;
  const uint64_t* sorted = L.sorted;
  const double zmax = (double)composite_z(sorted[0]);
  for (int i = t; i < n; i += BLOCK) {
    const double e = exp((double)composite_z(sorted[i]) - zmax);
    L.e[i] = e;
    L.cum[i] = e;
  }
  if (t == 0) {
    s.ints[0] = n;  // top-p survivors
    s.ints[1] = n;  // min-p survivors
  }
  __syncthreads();
  block_scan_array<BLOCK, (kFinalCap + BLOCK - 1) / BLOCK>(L.cum, n, s.red);
  if (a.top_p < 1.0f) {
    const double target = (double)a.top_p * L.cum[n - 1];
    for (int i = t; i < n; i += BLOCK)
      if (L.cum[i] >= target && (i == 0 || L.cum[i - 1] < target)) s.ints[0] = i + 1;
  }
  __syncthreads();
  const int lp = s.ints[0];
  if (a.min_p > 0.0f) {
    const double mp = (double)a.min_p;
    for (int i = t; i < lp; i += BLOCK)
      if (L.e[i] < mp && (i == 0 || L.e[i - 1] >= mp)) s.ints[1] = i;
  }
  __syncthreads();
  const int kept = s.ints[1] < lp ? s.ints[1] : lp;
  for (int i = t; i < kept; i += BLOCK)
    L.byid[i] = ((uint64_t)(uint32_t)composite_id(sorted[i]) << 32) | (uint32_t)i;
  __syncthreads();
  block_sort_asc<BLOCK>(L.byid, kept);
  for (int i = t; i < kept; i += BLOCK) L.cum[i] = L.e[(uint32_t)L.byid[i]];
  __syncthreads();
  block_scan_array<BLOCK, (kFinalCap + BLOCK - 1) / BLOCK>(L.cum, kept, s.red);
  const double E = L.cum[kept - 1];
  const double target = (double)a.uniforms[row] * E;
  if (t == 0) s.ints[2] = kept - 1;  // no C_j > u through rounding: the last kept id
  __syncthreads();
  for (int i = t; i < kept; i += BLOCK)
    if (L.cum[i] > target && (i == 0 || !(L.cum[i - 1] > target))) s.ints[2] = i;
  __syncthreads();
  if (t == 0) a.out_ids[row] = (int32_t)(L.byid[s.ints[2]] >> 32);
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = t; i < kept; i += BLOCK) prow[L.byid[i] >> 32] = (float)(L.e[(uint32_t)L.byid[i]] / E);
  }
}

// Finish one row from nl sorted non-history candidate lists (lists[s.off[l]], s.cnt[l]):
// add the history ids, select top-k or the min-p band exactly, and draw. Falls back to
// the row solver if a list overflowed. Every thread of the block calls it.
template <int BLOCK, int DT, bool MODE_K>
__device__ void finish_row(const Args& a, int row, const uint64_t* lists, int nl, uint32_t flags, Lds& L,
                           FinishShared& s) {
  const int t = threadIdx.x;
  if (t == 0) s.flags = flags;
  gather_prefixes<BLOCK, MODE_K>(a, lists, nl, L, s);
  if (a.H > 0) history_candidates<BLOCK, DT, MODE_K>(a, row, L, s);
  __syncthreads();
  flags = s.flags;
  if (flags & kFlagBadHistory) {
    if (t == 0) a.out_ids[row] = ARBOR_ID_BAD_HISTORY;
    return;
  }
  if (flags & kFlagInvalid) {
    if (t == 0) a.out_ids[row] = ARBOR_ID_INVALID;
    return;
  }
  if ((flags & kFlagOverflow) || s.uni_over) {
    __syncthreads();
    solve_row<BLOCK, DT>(a, row, L.htab, *L.ssh);
    return;
  }
  int n = s.n_uni;
  if (n == 0) {
    if (t == 0) a.out_ids[row] = ARBOR_ID_EMPTY;
    return;
  }
  if (MODE_K) {
    if (t < kWave) {
      // radix histogram in the last 1 KB of region A (wave buffers / chunk lists are consumed)
      if (n > a.top_k)
        wave_keep_topk<kFinalCap>(L.uni, n, a.top_k, reinterpret_cast<uint32_t*>(L.wbuf + kWaves * kWaveCap - 128));
      wave_sort_desc<kFinalCap>(L.uni, n);
      for (int i = t; i < n; i += kWave) L.sorted[i] = L.uni[i];
      if (t == 0) s.ints[3] = n;
    }
    __syncthreads();
    n = s.ints[3];
  } else {
    // band of the row's best z (a history id may be the best), then sort best first
    float m = -INFINITY;
    for (int i = t; i < n; i += BLOCK) m = fmaxf(m, composite_z(L.uni[i]));
    m = block_reduce_max<BLOCK, float>(m, reinterpret_cast<float*>(s.red));
    const float thr = m + a.ln_min_p_lo;
    if (t == 0) s.ints[3] = 0;
    __syncthreads();
    for (int i = t; i < n; i += BLOCK) {
      const uint64_t c = L.uni[i];
      if (composite_z(c) >= thr) L.sorted[atomicAdd(&s.ints[3], 1)] = ~c;
    }
    __syncthreads();
    n = s.ints[3];
    block_sort_asc<BLOCK>(L.sorted, n);
    for (int i = t; i < n; i += BLOCK) L.sorted[i] = ~L.sorted[i];
    __syncthreads();
  }
  finalize_candidates<BLOCK>(a, row, n, L, s);
}

}  // namespace arbor
