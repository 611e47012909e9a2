// row_solver.hpp -- the exact fallback: one workgroup solves one row.
//
// z is recomputed from the logits on every pass (tempered, masked, penalised from the
// LDS history table), so the solver needs no workspace; each cut (top-k by count, top-p by
// probability mass) is found by an MSB-first radix select on the 64-bit rank key (z
// descending, id ascending); the draw is a block scan in id order. Mass is fixed point
// (2^-40), so every sum is exact and independent of reduction order. Used for rows with
// more tied entries at a cut than the histogram solvers rank directly, and for streamed
// rows whose candidate list could not hold the answer.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"

namespace arbor {

// ---------------------------------------------------------------------------------------
// Row solver
// ---------------------------------------------------------------------------------------
struct SolverShared {
  uint64_t hist_w[256];
  uint32_t hist_c[256];
  uint64_t red64[kWaves];
  uint32_t red32[kWaves];
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
template <int BLOCK, typename ZAt>
__device__ CutResult radix_cut(ZAt zat, int V, float zmax, bool by_mass, uint64_t target,
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
      const float v = zat(i);
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
// 1 << a.hash_bits slots of LDS (when the row has a history).
template <int BLOCK, int DT>
__device__ __forceinline__ void solve_row(const Args& a, int row, uint32_t* htab, SolverShared& sh) {
  const int t = threadIdx.x;
  const int V = a.V;
  const void* xrow = row_ptr<DT>(a, row);
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
  __syncthreads();  // the history table is complete
  // 2. z of id i, recomputed from the logits on every pass: tempered, masked (-inf), and
  // penalised when i is a history id (the table probe ends at the first empty slot)
  const bool hist = a.H > 0;
  auto zat = [&](int i) -> float {
    if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) return -INFINITY;
    const float v = Elem<DT>::one(xrow, i) * a.inv_t + 0.0f;
    if (hist) {
      const uint32_t c = hist_count(htab, (uint32_t)a.hash_bits, (uint32_t)i);
      if (c) return penalize(v, c, a.pen);
    }
    return v;
  };
  // 3. row statistics
  uint32_t kmax = 0, kmin = 0xFFFFFFFFu, nf = 0;
  for (int i = t; i < V; i += BLOCK) {
    const float v = zat(i);
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
    const CutResult ck = radix_cut<BLOCK>(zat, V, zmax, false, (uint64_t)a.top_k, 0.0, kmax, kmin, sh);
    cut = ck.cut;
  }
  if (a.top_p < 1.0f) {
    CutResult cp;
    if (cut != 0ull) {
      // mass of the top-k survivors
      uint64_t m = 0;
      for (int i = t; i < V; i += BLOCK) {
        const float v = zat(i);
        if (v != -INFINITY && composite(v, i) >= cut) m += mass_fixed(rel_exp(v, zmax));
      }
      m = block_reduce_sum<BLOCK, uint64_t>(m, sh.red64);
      const double tg = ceil((double)a.top_p * (double)m);
      uint64_t target = tg < 1.0 ? 1ull : (uint64_t)tg;
      if (target > m) target = m;
      cp = radix_cut<BLOCK>(zat, V, zmax, true, target, 0.0, kmax, kmin, sh);
    } else {
      cp = radix_cut<BLOCK>(zat, V, zmax, true, 0ull, (double)a.top_p, kmax, kmin, sh);
    }
    if (cp.cut > cut) cut = cp.cut;
  }
  const bool use_min_p = a.min_p > 0.0f;

  // 6. kept mass and last kept id
  uint64_t E = 0;
  int32_t last = -1;
  for (int i = t; i < V; i += BLOCK) {
    const float v = zat(i);
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
        const float v = zat(i);
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
  if (t == 0) {
    const int32_t pick = sh.b32[2] >= 0 ? sh.b32[2] : last;
    a.out_ids[row] = pick;
    ring_append(a, row, pick);  // the row's history was read in step 1, before the barriers
  }
}

}  // namespace arbor
