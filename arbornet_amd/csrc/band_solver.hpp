// band_solver.hpp -- min-p as the only filter, for a row whose band (the ids with
// exp(z - zmax) >= min_p) is longer than the streaming kernel's 64-entry list. One
// workgroup per row, called by the streaming kernel's workgroup that found the overflow
// (the row is then still in the caches) or by the finishing kernel of a split row.
//
// Min-p alone needs no ranking: the kept set is every id in the band and the draw walks
// it in ascending id order. So one pass over the row suffices once zmax is known (the
// caller's list top is the row's maximum unless candidates were lost; the pass checks that
// and repeats itself with the maximum it found otherwise):
//  - every lane takes 8 consecutive ids per tile (two fp32 or one bf16 16-byte unit), with
//    the next three tiles in flight; a wave's 512 ids of a tile form one segment, and
//    segments are numbered in id order (tile * waves + wave);
//  - each id's final z is compared with zmax + ln(min_p) - 1e-3 in fp32 (penalties are
//    looked up only for ids that could pass, unless a penalty may raise z); the few that
//    pass get the band test in fp64, (double)z - zmax >= ln(min_p) (the contract's
//    exp((double)z - zmax) >= min_p, up to the rounding of exp and ln), and their mass
//    exp(z - zmax) in fp32 with the subtraction's rounding folded back (rel_exp), summed
//    in fp64;
//  - a segment's kept mass is the inclusive scan over its lanes of each lane's sequential
//    sum, so that the draw's rescan of one segment reproduces it bit for bit.
// The draw: prefix sums over the segments (one wave, in order), the segment where the
// running mass passes u * E, and a rescan of its 512 ids. Results do not depend on timing.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"
#include "row_solver.hpp"

namespace arbor {

constexpr int kBandIds = 8;  // consecutive ids per lane per tile
constexpr int kBandDepth = 4;  // tiles a lane has requested ahead of the one it processes

struct BandShared {
  double redd[kWaves];
  uint32_t red32[kWaves];
  int32_t red_i[kWaves];
  double P;      // prefix mass before the crossing segment
  int seg;       // the crossing segment (-1: none)
  int32_t pick;  // the drawn id (-1: none yet)
};

// Segments of a row of V ids drawn by a workgroup of BLOCK threads.
__host__ __device__ constexpr int band_segments(int V, int block) {
  return (V + block * kBandIds - 1) / (block * kBandIds) * (block / kWave);
}
// LDS the band solver needs beside the history table: its shared block and one double per
// segment.
__host__ __device__ constexpr size_t band_lds_bytes(int V, int block) {
  return (sizeof(BandShared) + 15) / 16 * 16 + sizeof(double) * (size_t)band_segments(V, block);
}

// 16-byte unit of raw words at id e0 (a multiple of the unit's ids). WHOLE: the row is
// aligned and made of whole units, so a unit is entirely inside the row or entirely past
// its end (then it holds -inf); otherwise element loads, -inf past the end.
template <int DT, bool WHOLE>
__device__ __forceinline__ void band_load(const void* row, int e0, int V, uint32_t* w) {
  if constexpr (WHOLE) {
    if (e0 < V) {
      typedef unsigned int u4 __attribute__((ext_vector_type(4)));
      const u4 v = *reinterpret_cast<const u4*>(static_cast<const char*>(row) + (size_t)e0 * Elem<DT>::kBytes);
      w[0] = v.x;
      w[1] = v.y;
      w[2] = v.z;
      w[3] = v.w;
    } else {
      const uint32_t ninf = DT == ARBOR_DTYPE_F32 ? 0xFF800000u : 0xFF80FF80u;
      w[0] = w[1] = w[2] = w[3] = ninf;
    }
  } else {
    load_raw<DT>(row, e0, V, false, w);
  }
}

// ALIGNED: rows of whole aligned 16-byte units (the caller checks).
template <int BLOCK, int DT, bool ALIGNED>
__device__ __forceinline__ void solve_band_row(const Args& a, int row, uint32_t top_key, uint32_t* htab,
                                               unsigned char* lds) {
  constexpr int W = kBandIds / Elem<DT>::kVec;  // 16-byte units per lane per tile
  constexpr int WORDS = 4 * W;                  // raw dwords per lane per tile
  constexpr int WAVES = BLOCK / kWave;
  constexpr int TILE = BLOCK * kBandIds;
  BandShared& sh = *reinterpret_cast<BandShared*>(lds);
  double* seg = reinterpret_cast<double*>(lds + (sizeof(BandShared) + 15) / 16 * 16);
  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  const int V = a.V;
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = a.mask ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const int ntiles = (V + TILE - 1) / TILE;
  const int nseg = ntiles * WAVES;

  // history table of the whole row, with occurrence counts
  uint32_t flags = 0;
  if (a.H > 0) {
    const int P = 1 << a.hash_bits;
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
  __syncthreads();
  const bool hist = a.H > 0;
  const bool probe_all = hist && !a.pen_mono;  // a penalty may raise z: every id is looked up

  // z of the 8 ids of a lane's tile, from raw words; masked ids are -inf whatever their value.
  // With penalties that never raise z, only ids whose unpenalised z reaches thr are looked
  // up (the others stay below thr, and below the maximum, either way); `full` looks up all.
  auto final_z = [&](const uint32_t* w, int base, float thr, bool full, float* z) {
    uint32_t mbits = 0xFFu;
    if (mrow && base < V) mbits = (mrow[base >> 5] >> (base & 31)) & 0xFFu;
#pragma unroll
    for (int j = 0; j < kBandIds; ++j) {
      float v = unpack_unit<DT>(w, j) * a.inv_t + 0.0f;
      if (!((mbits >> j) & 1u)) v = -INFINITY;
      if (hist && base + j < V && (full || v >= thr)) {
        const uint32_t c = hist_count(htab, (uint32_t)a.hash_bits, (uint32_t)(base + j));
        if (c) v = penalize(v, c, a.pen);
      }
      z[j] = v;
    }
  };

  uint32_t kmax = 0;
  int32_t last = -1;
  bool any = false;
  for (int attempt = 0; attempt < 2; ++attempt) {
    // top_key 0: the maximum is not known yet; this pass only finds it
    const float zh = top_key ? key_value(top_key) : -INFINITY;
    const double zhd = (double)zh;
    // With the maximum known and penalties that only lower z, an id whose tempered z is
    // below zh + ln(min_p) - 1e-3 can be neither in the band nor above the maximum, so one
    // multiply and one compare settle most ids. Otherwise every finite id is looked at.
    const bool full = probe_all || !top_key;
    const float thr = full ? -FLT_MAX : zh + a.ln_min_p_lo;
    const float band_thr = zh + a.ln_min_p_lo;
    uint32_t buf[kBandDepth][WORDS];
    auto request = [&](int tile, uint32_t* w) {
      const int base = tile * TILE + wave * (kWave * kBandIds) + lane * kBandIds;
#pragma unroll
      for (int u = 0; u < W; ++u) band_load<DT, ALIGNED>(xrow, base + u * Elem<DT>::kVec, V, w + 4 * u);
    };
#pragma unroll
    for (int d = 0; d < kBandDepth; ++d)
      if (d < ntiles) request(d, buf[d]);
    uint32_t lk = 0;
    bool bad = false, fin = top_key != 0u;  // a known maximum is a finite id of the row
    int32_t lst = -1;
    for (int tb = 0; tb < ntiles; tb += kBandDepth) {
#pragma unroll
      for (int d = 0; d < kBandDepth; ++d) {
        const int tile = tb + d;
        if (tile >= ntiles) break;
        const int base = tile * TILE + wave * (kWave * kBandIds) + lane * kBandIds;
        float v[kBandIds];
        uint32_t cbits = 0u;  // the lane's ids at or above thr
#pragma unroll
        for (int j = 0; j < kBandIds; ++j) {
          v[j] = unpack_unit<DT>(buf[d], j) * a.inv_t + 0.0f;
          cbits |= (v[j] >= thr ? 1u : 0u) << j;
        }
        if (tile + kBandDepth < ntiles) request(tile + kBandDepth, buf[d]);
        uint32_t mbits = 0xFFu;
        if (full) {  // NaN passes no threshold: detected here (masked ids are -inf whatever they hold)
          if (mrow && base < V) mbits = (mrow[base >> 5] >> (base & 31)) & 0xFFu;
#pragma unroll
          for (int j = 0; j < kBandIds; ++j) bad |= ((mbits >> j) & 1u) && v[j] != v[j];
        }
        double s = 0.0;
        bool kept_any = false;
        if (__ballot(cbits != 0u)) {
          if (!full && mrow && base < V) mbits = (mrow[base >> 5] >> (base & 31)) & 0xFFu;
          cbits &= mbits;
          // each lane's candidates in ascending id order (the order of the rescan's sums),
          // as many rounds as the lane with the most
          while (__ballot(cbits != 0u)) {
            if (cbits) {
              const int j = __builtin_ctz(cbits);
              cbits &= cbits - 1u;
              float z = v[0];
#pragma unroll
              for (int q = 1; q < kBandIds; ++q) z = j == q ? v[q] : z;
              const int id = base + j;
              if (hist && id < V) {
                const uint32_t c = hist_count(htab, (uint32_t)a.hash_bits, (uint32_t)id);
                if (c) z = penalize(z, c, a.pen);
              }
              if (is_invalid(z)) {
                bad = true;
              } else if (z != -INFINITY) {
                fin = true;
                // the maximum: tracked where the known one may be exceeded
                if (full || z > zh) {
                  const uint32_t k = order_key(z);
                  lk = k > lk ? k : lk;
                }
                if (top_key && z >= band_thr && (double)z - zhd >= a.ln_min_p) {
                  s += (double)rel_exp(z, zh);
                  kept_any = true;
                  lst = id;
                }
              }
            }
          }
        }
        // the segment's mass: the inclusive scan over lanes of the lanes' sequential sums
        double incl = 0.0;
        if (__ballot(kept_any)) incl = wave_scan_incl(s);
        if (lane == kWave - 1) seg[tile * WAVES + wave] = incl;
      }
    }
    kmax = block_reduce_max<BLOCK, uint32_t>(lk, sh.red32);
    flags |= bad ? kFlagInvalid : 0u;
    flags = block_reduce_max<BLOCK, uint32_t>(flags & kFlagBadHistory ? 2u : (flags & kFlagInvalid ? 1u : 0u),
                                              sh.red32);
    any = block_reduce_max<BLOCK, uint32_t>(fin ? 1u : 0u, sh.red32) != 0u;
    last = block_reduce_max<BLOCK, int32_t>(lst, sh.red_i);
    // the band was measured from the row's maximum: done (a list top below the maximum,
    // or none, takes a second pass from the maximum just found)
    if (flags != 0 || !any || (top_key && kmax <= top_key)) break;
    top_key = kmax;
  }
  float* prow = a.write_probs ? a.out_probs + (size_t)row * (size_t)V : nullptr;
  if (flags != 0 || !any) {
    if (t == 0) a.out_ids[row] = flags == 2u ? ARBOR_ID_BAD_HISTORY : (flags == 1u ? ARBOR_ID_INVALID : ARBOR_ID_EMPTY);
    if (prow)
      for (int i = t; i < V; i += BLOCK) prow[i] = 0.0f;
    return;
  }
  const float zh = key_value(top_key);  // the maximum the passes measured the band from
  const double zhd = (double)zh;
  const float thr = zh + a.ln_min_p_lo;

  // prefix sums over the segments in id order (wave 0), the total E and the crossing
  // segment: the first whose end passes u * E
  const float u = a.uniforms[row];
  if (wave == 0) {
    double carry = 0.0;
    for (int c = 0; c < nseg; c += kWave) {
      const double v = c + lane < nseg ? seg[c + lane] : 0.0;
      const double incl = wave_scan_incl(v) + carry;
      if (c + lane < nseg) seg[c + lane] = incl;  // running mass at the segment's end
      carry = lane_get(incl, kWave - 1);
    }
    const double target = (double)u * carry;
    int found = -1;
    for (int c = 0; c < nseg && found < 0; c += kWave) {
      const uint64_t over = __ballot(c + lane < nseg && seg[c + lane] > target);
      if (over) found = c + __ffsll((long long)over) - 1;
    }
    if (lane == 0) {
      sh.seg = found;
      sh.P = found > 0 ? seg[found - 1] : 0.0;
      sh.redd[0] = carry;
      sh.pick = -1;
    }
  }
  __syncthreads();
  const double E = sh.redd[0];
  const int sx = sh.seg;
  if (sx >= 0 && wave == sx % WAVES) {
    // rescan the crossing segment: the same lane sums, in id order
    const int tile = sx / WAVES;
    const int base = tile * TILE + wave * (kWave * kBandIds) + lane * kBandIds;
    uint32_t w[WORDS];
#pragma unroll
    for (int uu = 0; uu < W; ++uu) band_load<DT, ALIGNED>(xrow, base + uu * Elem<DT>::kVec, V, w + 4 * uu);
    float z[kBandIds];
    final_z(w, base, thr, probe_all, z);
    double e[kBandIds];
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kBandIds; ++j) {
      e[j] = 0.0;
      if (z[j] >= thr && (double)z[j] - zhd >= a.ln_min_p) e[j] = (double)rel_exp(z[j], zh);
      s += e[j];
    }
    const double incl = wave_scan_incl(s);
    const double excl = lane_shift_down(incl, 0.0);
    const double target = (double)u * E - sh.P;
    // the lane whose running mass passes the target, then the id inside it (none through
    // rounding: the segment's last lane with a kept id)
    const uint64_t over = __ballot(incl > target);
    const uint64_t has = __ballot(s > 0.0);
    if (over || has) {
      const int l = over ? __ffsll((long long)over) - 1 : 63 - __builtin_clzll(has);
      if (lane == l) {
        double run = excl;
        int32_t p = -1, lastw = -1;
#pragma unroll
        for (int j = 0; j < kBandIds; ++j) {
          if (e[j] > 0.0) lastw = base + j;
          run += e[j];
          if (p < 0 && e[j] > 0.0 && run > target) p = base + j;
        }
        sh.pick = p >= 0 ? p : lastw;  // rounding inside the lane: its last kept id
      }
    }
  }
  __syncthreads();
  const int32_t pick = sh.pick >= 0 ? sh.pick : last;  // no crossing (u * E rounds to E): the last kept id
  if (prow) {
    for (int i0 = t * kBandIds; i0 < V; i0 += BLOCK * kBandIds) {
      uint32_t w[WORDS];
#pragma unroll
      for (int uu = 0; uu < W; ++uu) band_load<DT, ALIGNED>(xrow, i0 + uu * Elem<DT>::kVec, V, w + 4 * uu);
      float z[kBandIds];
      final_z(w, i0, thr, probe_all, z);
#pragma unroll
      for (int j = 0; j < kBandIds; ++j) {
        if (i0 + j >= V) break;
        float q = 0.0f;
        if (z[j] >= thr && (double)z[j] - zhd >= a.ln_min_p) q = (float)((double)rel_exp(z[j], zh) / E);
        prow[i0 + j] = q;
      }
    }
  }
  if (t == 0) {
    a.out_ids[row] = pick;
    ring_append(a, row, pick);  // the row's history was read into the table before the passes
  }
}

// LDS of draw_band_candidates: ids, masses and ids in id order (BLOCK each) and the
// block reductions' scratch.
template <int BLOCK>
__host__ __device__ constexpr size_t band_draw_lds_bytes() {
  return 3 * sizeof(uint32_t) * BLOCK + (sizeof(double) + sizeof(int32_t)) * (BLOCK / kWave);
}

// Min-p draw over a row's candidates when every id of the band is among them: cand[0, n)
// (n <= BLOCK) holds final-z composites of distinct ids, top_key is the order key of the
// row's maximum z, and the row's probabilities are zero where the draw writes none. Band
// membership and masses are those of solve_band_row; each member's place in id order is
// the count of members with smaller ids, and the masses, placed in that order, are summed
// by one block scan, so the result does not depend on the candidates' order.
template <int BLOCK>
__device__ __forceinline__ void draw_band_candidates(const Args& a, int row, const uint64_t* cand, int n, uint32_t top_key, float u,
                                     unsigned char* lds) {
  uint32_t* ids = reinterpret_cast<uint32_t*>(lds);  // [BLOCK] member ids, 0xFFFFFFFF elsewhere
  float* es = reinterpret_cast<float*>(ids + BLOCK);  // [BLOCK] masses in id order
  int32_t* sid = reinterpret_cast<int32_t*>(es + BLOCK);  // [BLOCK] ids in id order
  double* red_d = reinterpret_cast<double*>(sid + BLOCK);
  int32_t* red_i = reinterpret_cast<int32_t*>(red_d + BLOCK / kWave);
  const int t = threadIdx.x;
  const float zh = key_value(top_key);
  const double zhd = (double)zh;
  const float thr = zh + a.ln_min_p_lo;
  const uint64_t c = t < n ? cand[t] : 0ull;
  const float z = composite_z(c);
  const int32_t id = composite_id(c);
  const bool in = c != 0ull && z >= thr && (double)z - zhd >= a.ln_min_p;
  ids[t] = in ? (uint32_t)id : 0xFFFFFFFFu;
  const int nb = block_reduce_sum<BLOCK, int32_t>(in ? 1 : 0, red_i);  // its barriers publish ids
  const float e = in ? rel_exp(z, zh) : 0.0f;
  if (in) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const u4* v = reinterpret_cast<const u4*>(ids);
    const uint32_t me = (uint32_t)id;
    int rank = 0;
    for (int j = 0; j < (n + 3) / 4; ++j) {
      const u4 w = v[j];
      rank += (w.x < me ? 1 : 0) + (w.y < me ? 1 : 0) + (w.z < me ? 1 : 0) + (w.w < me ? 1 : 0);
    }
    es[rank] = e;
    sid[rank] = id;
  }
  __syncthreads();
  const double ev = t < nb ? (double)es[t] : 0.0;
  double E;
  const double incl = block_scan_excl<BLOCK, double>(ev, red_d, &E) + ev;
  const double target = (double)u * E;
  // the first member in id order whose running mass passes u * E (none through rounding at
  // u -> 1: the last member)
  const int first = block_reduce_min<BLOCK, int32_t>(t < nb && incl > target ? t : BLOCK, red_i);
  if (t == 0) {
    const int32_t pick = sid[first < nb ? first : nb - 1];
    a.out_ids[row] = pick;
    ring_append(a, row, pick);
  }
  if (a.write_probs && in) a.out_probs[(size_t)row * (size_t)a.V + id] = (float)((double)e / E);
}

}  // namespace arbor
