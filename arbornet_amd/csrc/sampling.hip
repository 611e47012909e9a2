// sampling.hip -- MI355X (gfx950) token-sampling kernels and the extern "C" ABI of
// libarbor_hip.so (declared in include/arbor_sampling.h).
//
// Two device paths compute the same contract:
//
//  * streaming path (top-k <= 64, or min-p as the only filter). One 1024-thread
//    workgroup per compute unit streams a row (or, when the batch is smaller than the
//    chip, one chunk of a row) from HBM exactly once with 16-byte loads, 8 loads in
//    flight per lane. Temperature and the allow-mask are applied in registers; ids that
//    occur in the row's history are skipped through an LDS bitmap and evaluated exactly
//    once per row at the end. Each wave keeps a private LDS list of candidates above a
//    running threshold: the k-th best of the 64 lane maxima of every 2048-element batch
//    (a lower bound of the k-th best seen so far), tightened by an exact wave radix select
//    when the list fills. The row is finished from at most 1024 candidates in fp64
//    (top-k, top-p, min-p, inverse-CDF draw in id order), in the same workgroup when the
//    row was not split, else by finish_kernel from the chunks' published lists.
//
//  * row solver (top-p without top-k, plain sampling, top-k > 64, or a streamed row whose
//    candidate list overflowed): see row_solver.hpp.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <cmath>

#include "../../include/arbor_sampling.h"
#include "args.hpp"
#include "block_ops.hpp"
#include "candidates.hpp"
#include "row_solver.hpp"
#include "topk_path.hpp"

namespace arbor {

template <int DT>
__global__ void __launch_bounds__(kBlock) solver_kernel(Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SolverShared sh;
  solve_row<kBlock, DT>(a, blockIdx.x, reinterpret_cast<uint32_t*>(smem), sh);
}

template <int DT, bool PEN, bool MASK, bool MODE_K, bool INLINE>
__global__ void __launch_bounds__(kBlock) stream_kernel(Args a) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int kUnroll = Elem<DT>::kUnroll;
  extern __shared__ __align__(16) unsigned char smem[];
  Lds L(smem);
  __shared__ FinishShared s;
  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  const int row = blockIdx.x / a.S, chunk = blockIdx.x % a.S;
  const int c0 = chunk * a.chunk_len;
  const int c1 = min(a.V, c0 + a.chunk_len);
  const void* xrow = row_ptr<DT>(a, row);

  if (t == 0) {
    s.flags = 0u;
    s.next_batch = 0;
  }
  if (PEN) {
    for (int i = t; i < a.bitmap_words; i += kBlock) L.bitmap[i] = 0u;
    __syncthreads();
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    for (int j = t; j < a.H; j += kBlock) {
      const int32_t id = h[j];
      if (id >= c0 && id < c1) atomicOr(&L.bitmap[(id - c0) >> 5], 1u << ((id - c0) & 31));
    }
  }
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = c0 + t; i < c1; i += kBlock) prow[i] = 0.0f;
  }
  __syncthreads();

  // ---- stream the chunk ----
  // Double-buffered: the loads of batch i+1 are in flight while batch i is processed.
  uint64_t* buf = L.wbuf + wave * kWaveCap;
  uint32_t* rh = L.whist + wave * 256;
  int wc = 0;
  float thr = -FLT_MAX;  // accept z >= thr; -inf is never a candidate
  bool bad = false, ovf = false;
  const uint32_t* mrow = MASK ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const bool aligned = a.aligned != 0;
  const int n_units = (c1 - c0 + VEC - 1) / VEC;

  struct Batch {
    float z[kUnroll][VEC];
    uint32_t mw[kUnroll];
  };
  auto load = [&](int ub, Batch& bt) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int e0 = c0 + (ub + u * kWave + lane) * VEC;
      load_unit<DT>(xrow, e0, c1, aligned, bt.z[u]);
      if (MASK) bt.mw[u] = e0 < c1 ? mrow[e0 >> 5] : 0u;
    }
  };
  // returns false when the wave's list overflowed (min-p band only)
  auto process = [&](int ub, Batch& bt) -> bool {
    float lmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int e0 = c0 + (ub + u * kWave + lane) * VEC;
      const uint32_t mb = MASK ? bt.mw[u] >> (e0 & 31) : ~0u;
      const uint32_t pb = PEN && e0 < c1 ? L.bitmap[(e0 - c0) >> 5] >> ((e0 - c0) & 31) : 0u;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        float v = bt.z[u][j] * a.inv_t;
        if (PEN && ((pb >> j) & 1u)) v = -INFINITY;  // history id: evaluated at the finish
        if (MASK && !((mb >> j) & 1u)) v = -INFINITY;
        const bool iv = is_invalid(v);
        bad |= iv;
        v = iv ? -INFINITY : v;
        lmax = fmaxf(lmax, v);
        bt.z[u][j] = v;
      }
    }
    // raise the threshold from this batch's lane maxima
    if (MODE_K) {
      const uint32_t key = wave_sort64_desc_u32(order_key(lmax));
      thr = fmaxf(thr, key_value(__shfl(key, a.top_k - 1)));
    } else {
      const float m = wave_max(lmax);
      if (m > -INFINITY) thr = fmaxf(thr, m + a.ln_min_p_lo);
    }
    int c = 0;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int j = 0; j < VEC; ++j) c += bt.z[u][j] >= thr ? 1 : 0;
    int cnt = wave_sum(c);
    if (cnt == 0) return true;
    if (wc + cnt > kWaveCap) {
      if (MODE_K) {
        if (wc > a.top_k) thr = fmaxf(thr, wave_keep_topk<kWaveCap>(buf, wc, a.top_k, rh));
      } else if (wc > 0) {
        thr = fmaxf(thr, wave_keep_band<kWaveCap>(buf, wc, a.ln_min_p_lo));
      }
      c = 0;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int j = 0; j < VEC; ++j) c += bt.z[u][j] >= thr ? 1 : 0;
      cnt = wave_sum(c);
    }
    if (wc + cnt <= kWaveCap) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int e0 = c0 + (ub + u * kWave + lane) * VEC;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const bool take = bt.z[u][j] >= thr;
          const uint64_t bal = __ballot(take);
          if (bal) {
            if (take) buf[wc + lanes_below(bal)] = composite(bt.z[u][j] + 0.0f, e0 + j);
            wc += __popcll(bal);
          }
        }
      }
      return true;
    }
    // a batch larger than the buffer: append 64 at a time, pruning in between
#pragma unroll 1
    for (int q = 0; q < kUnroll * VEC; ++q) {
      float v = -INFINITY;
#pragma unroll
      for (int uu = 0; uu < kUnroll; ++uu)
#pragma unroll
        for (int jj = 0; jj < VEC; ++jj)
          if (uu * VEC + jj == q) v = bt.z[uu][jj];
      const int id = c0 + (ub + (q / VEC) * kWave + lane) * VEC + (q % VEC);
      if (!__ballot(v >= thr)) continue;
      if (wc + kWave > kWaveCap) {
        if (MODE_K)
          thr = fmaxf(thr, wave_keep_topk<kWaveCap>(buf, wc, a.top_k, rh));
        else
          thr = fmaxf(thr, wave_keep_band<kWaveCap>(buf, wc, a.ln_min_p_lo));
        if (wc + kWave > kWaveCap) return false;
      }
      const bool take = v >= thr;
      const uint64_t bal = __ballot(take);
      if (take) buf[wc + lanes_below(bal)] = composite(v + 0.0f, id);
      wc += __popcll(bal);
    }
    return true;
  };

  // batches are handed out from an LDS counter, so faster waves take more of them
  constexpr int kBatch = kUnroll * kWave;  // units per batch
  const int n_batches = (n_units + kBatch - 1) / kBatch;
  auto grab = [&]() -> int {
    int b = 0;
    if (lane == 0) b = atomicAdd(&s.next_batch, 1);
    return __shfl(b, 0);
  };
  Batch ba, bb;
  int bi = grab();
  if (bi < n_batches) load(bi * kBatch, ba);
  while (bi < n_batches) {
    int bn = grab();
    if (bn < n_batches) load(bn * kBatch, bb);
    if (!process(bi * kBatch, ba)) {
      ovf = true;
      break;
    }
    bi = bn;
    if (bi >= n_batches) break;
    bn = grab();
    if (bn < n_batches) load(bn * kBatch, ba);
    if (!process(bi * kBatch, bb)) {
      ovf = true;
      break;
    }
    bi = bn;
  }
  // final wave list: exact top-k (or the band of the wave's best), sorted best first
  if (!ovf) {
    if (MODE_K) {
      if (wc > a.top_k) wave_keep_topk<kWaveCap>(buf, wc, a.top_k, rh);
    } else if (wc > 0) {
      wave_keep_band<kWaveCap>(buf, wc, a.ln_min_p_lo);
    }
    wave_sort_desc<kWaveCap>(buf, wc);
  }
  if (__ballot(bad) && lane == 0) atomicOr(&s.flags, kFlagInvalid);
  if (ovf && lane == 0) atomicOr(&s.flags, kFlagOverflow);
  if (lane == 0) {
    s.cnt[wave] = ovf ? 0 : wc;
    s.off[wave] = wave * kWaveCap;
  }
  __syncthreads();

  if (INLINE) {
    finish_row<kBlock, DT, MODE_K>(a, row, L.wbuf, kWaves, s.flags, L, s);
    return;
  }
  // ---- publish this chunk's list for finish_kernel ----
  gather_prefixes<kBlock, MODE_K>(a, L.wbuf, kWaves, L, s);
  if (t < kWave) {
    const size_t slot = (size_t)row * (size_t)a.S + (size_t)chunk;
    int n = s.n_uni;
    uint32_t fl = s.flags | (s.uni_over ? kFlagOverflow : 0u);
    if (!(fl & kFlagOverflow)) {
      if (MODE_K) {
        if (n > a.top_k)
          wave_keep_topk<kFinalCap>(L.uni, n, a.top_k, reinterpret_cast<uint32_t*>(L.wbuf + kWaves * kWaveCap - 128));
      } else if (n > kChunkSlot) {
        fl |= kFlagOverflow;
      }
    }
    if (!(fl & kFlagOverflow)) {
      wave_sort_desc<kFinalCap>(L.uni, n);
      uint64_t* dst = a.cand + slot * kChunkSlot;
      for (int i = lane; i < n; i += kWave) dst[i] = L.uni[i];
    }
    if (t == 0) {
      a.hdr[slot * 2 + 0] = (fl & kFlagOverflow) ? 0u : (uint32_t)n;
      a.hdr[slot * 2 + 1] = fl;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Streaming top-k (1 <= k <= 64): register-resident candidate lists, see topk_path.hpp
// ---------------------------------------------------------------------------------------
struct TopkShared {
  int next_batch;
  uint32_t flags;
  int cnt[kListSlots];
};

// Dynamic LDS of topk_kernel: per-wave scratch, list slots, history table, chunk bitmap.
__host__ __device__ constexpr size_t topk_lds_bytes(int hash_slots, int bitmap_words) {
  return sizeof(uint64_t) * ((size_t)kWaves * kWave + (size_t)kListSlots * kWave) +
         sizeof(uint32_t) * ((size_t)hash_slots + (size_t)bitmap_words);
}

template <int DT, bool PEN, bool MASK, bool INLINE>
__global__ void __launch_bounds__(kBlock) topk_kernel(Args a) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int U = Elem<DT>::kUnroll;
  constexpr int NQ = VEC * U;           // elements per lane per batch
  constexpr int kBatch = U * kWave;     // units per batch
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* scratch_all = reinterpret_cast<uint64_t*>(smem);
  uint64_t* lists = scratch_all + kWaves * kWave;
  uint32_t* htab = reinterpret_cast<uint32_t*>(lists + kListSlots * kWave);
  __shared__ TopkShared s;

  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  const int row = blockIdx.x / a.S, chunk = blockIdx.x % a.S;
  const int c0 = chunk * a.chunk_len;
  const int c1 = min(a.V, c0 + a.chunk_len);
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = MASK ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const bool own_hist = PEN && chunk == 0;  // this workgroup evaluates the row's history ids
  const bool hist_wave = own_hist && wave == kWaves - 1;
  uint32_t* bitmap = htab + (own_hist ? (1 << a.hash_bits) : 0);
  uint64_t* scr = scratch_all + wave * kWave;
  const bool aligned = a.aligned != 0;
  const int n_units = (c1 - c0 + VEC - 1) / VEC;
  const int n_batches = (n_units + kBatch - 1) / kBatch;
  const int k = a.top_k;

  struct Batch {
    uint32_t w[U][4];  // raw 16-byte units
    uint32_t mw[U];
  };
  auto load = [&](int bi, Batch& bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e0 = c0 + (bi * kBatch + u * kWave + lane) * VEC;
      load_raw<DT>(xrow, e0, c1, aligned, bt.w[u]);
      if (MASK) bt.mw[u] = e0 < c1 ? mrow[e0 >> 5] : 0u;
    }
  };

  // the first batch of every streaming wave is in flight during the setup
  Batch ba, bb;
  int bi = hist_wave ? n_batches : wave;
  if (bi < n_batches) load(bi, ba);
  int32_t hid[(ARBOR_HISTORY_MAX + kBlock - 1) / kBlock];
  if (PEN) {
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
#pragma unroll
    for (int r = 0; r < (ARBOR_HISTORY_MAX + kBlock - 1) / kBlock; ++r) {
      const int j = t + r * kBlock;
      hid[r] = j < a.H ? h[j] : -1;
    }
  }
  if (t == 0) {
    s.next_batch = own_hist ? kWaves - 1 : kWaves;
    s.flags = 0u;
    s.cnt[kListSlots - 1] = 0;
  }
  if (PEN) {
    for (int i = t; i < a.bitmap_words; i += kBlock) bitmap[i] = 0u;
    if (own_hist)
      for (int i = t; i < (1 << a.hash_bits); i += kBlock) htab[i] = kEmptySlot;
  }
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = c0 + t; i < c1; i += kBlock) prow[i] = 0.0f;
  }
  __syncthreads();
  if (PEN) {
    bool bad = false;
#pragma unroll
    for (int r = 0; r < (ARBOR_HISTORY_MAX + kBlock - 1) / kBlock; ++r) {
      const int32_t id = hid[r];
      if (id >= a.V) {
        bad = true;
      } else if (id >= 0) {
        if (id >= c0 && id < c1) atomicOr(&bitmap[(id - c0) >> 5], 1u << ((id - c0) & 31));
        if (own_hist) hist_insert(htab, (uint32_t)a.hash_bits, (uint32_t)id);
      }
    }
    if (bad) atomicOr(&s.flags, kFlagBadHistory);
  }
  __syncthreads();

  // ---- the row's history ids, penalised, as one more list (one wave) ----
  if (hist_wave) {
    uint64_t hbest = 0ull;
    float hthr = -FLT_MAX;
    bool inv = false;
    const int P = 1 << a.hash_bits;
    constexpr int M = 4;
    for (int s0 = 0; s0 < P; s0 += kWave * M) {
      int idq[M];
      uint32_t cq[M], mq[M];
      float xq[M], zq[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int slot = s0 + m * kWave + lane;
        const uint32_t e = slot < P ? htab[slot] : kEmptySlot;
        idq[m] = e != kEmptySlot ? (int)(e >> 12) : -1;
        cq[m] = (e & 4095u) + 1u;
        xq[m] = idq[m] >= 0 ? Elem<DT>::one(xrow, idq[m]) : 0.0f;
        mq[m] = (MASK && idq[m] >= 0) ? mrow[idq[m] >> 5] : ~0u;
      }
      uint32_t pend = 0u;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float z = -INFINITY;
        if (idq[m] >= 0) {
          z = penalize(xq[m] * a.inv_t + 0.0f, cq[m], a.pen);
          if (!((mq[m] >> (idq[m] & 31)) & 1u)) z = -INFINITY;
          if (is_invalid(z)) {
            inv = true;
            z = -INFINITY;
          }
        }
        zq[m] = z;
        if (z != -INFINITY && z >= hthr) pend |= 1u << m;
      }
      list_absorb<M>(hbest, hthr, k, pend, [&](int q) { return zq[q]; }, [&](int q) { return idq[q]; }, scr);
    }
    if (__ballot(inv) && lane == 0) atomicOr(&s.flags, kFlagInvalid);
    const int n = min(k, list_count(hbest));
    if (lane < n) lists[(kListSlots - 1) * kWave + lane] = hbest;
    if (lane == 0) s.cnt[kListSlots - 1] = n;
  }

  // ---- stream the chunk: batches handed out from an LDS counter, double-buffered ----
  uint64_t best = 0ull;
  float thr = -FLT_MAX;  // accept z >= thr
  bool bad = false;
  auto grab = [&]() -> int {
    int b = 0;
    if (lane == 0) b = atomicAdd(&s.next_batch, 1);
    return __shfl(b, 0);
  };
  auto process = [&](int b, Batch& bt) {
    const int ub = b * kBatch;
    // tempered logit of slot q; history ids and masked ids read as -inf (history ids are
    // in the history list), NaN / +inf are flagged and read as -inf
    auto zof = [&](int q) -> float {
      const int u = q / VEC, j = q % VEC;
      const int e0 = c0 + (ub + u * kWave + lane) * VEC;
      float v = unpack_unit<DT>(bt.w[u], j) * a.inv_t;
      if (PEN && e0 < c1 && ((bitmap[(e0 - c0) >> 5] >> (((e0 - c0) & 31) + j)) & 1u)) v = -INFINITY;
      if (MASK && !((bt.mw[u] >> ((e0 & 31) + j)) & 1u)) v = -INFINITY;
      return is_invalid(v) ? -INFINITY : v;
    };
    if (list_count(best) < k) {
      // until the list holds k entries: the k-th best lane maximum bounds this batch's k-th
      float lmax = -INFINITY;
#pragma unroll
      for (int q = 0; q < NQ; ++q) lmax = fmaxf(lmax, zof(q));
      const uint32_t key = wave_sort64_desc_u32(order_key(lmax));
      thr = fmaxf(thr, key_value(__shfl(key, k - 1)));
    }
    uint32_t pend = 0u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e0 = c0 + (ub + u * kWave + lane) * VEC;
      const uint32_t mb = MASK ? bt.mw[u] >> (e0 & 31) : ~0u;
      const uint32_t pb = PEN && e0 < c1 ? bitmap[(e0 - c0) >> 5] >> ((e0 - c0) & 31) : 0u;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float v = unpack_unit<DT>(bt.w[u], j) * a.inv_t;
        const bool skip = (PEN && ((pb >> j) & 1u)) || (MASK && !((mb >> j) & 1u));
        bad |= !skip && is_invalid(v);
        if (!skip && v >= thr && !is_invalid(v)) pend |= 1u << (u * VEC + j);
      }
    }
    list_absorb<NQ>(best, thr, k, pend, zof,
                    [&](int q) { return c0 + (ub + (q / VEC) * kWave + lane) * VEC + (q % VEC); }, scr);
  };
  if (hist_wave) {
    bi = grab();
    if (bi < n_batches) load(bi, ba);
  }
  while (bi < n_batches) {
    int bn = grab();
    if (bn < n_batches) load(bn, bb);
    process(bi, ba);
    bi = bn;
    if (bi >= n_batches) break;
    bn = grab();
    if (bn < n_batches) load(bn, ba);
    process(bi, bb);
    bi = bn;
  }
  {
    const int n = min(k, list_count(best));
    if (lane < n) lists[wave * kWave + lane] = best;
    if (lane == 0) s.cnt[wave] = n;
    if (__ballot(bad) && lane == 0) atomicOr(&s.flags, kFlagInvalid);
  }
  __syncthreads();

  // ---- tree merge of the lists; the result lands in slot 0 ----
  for (int m = kListSlots, st = 1; m > 1; st *= 2) {
    if (wave < m / 2) {
      const int ia = 2 * wave * st, ib = ia + st;
      const int na = s.cnt[ia], nb = s.cnt[ib];
      const uint64_t va = lane < na ? lists[ia * kWave + lane] : 0ull;
      const uint64_t vb = lane < nb ? lists[ib * kWave + lane] : 0ull;
      const uint64_t v = list_merge(va, vb);
      const int n = min(k, na + nb);
      wave_lds_sync();
      if (lane < n) lists[ia * kWave + lane] = v;
      if (lane == 0) s.cnt[ia] = n;
    }
    m = (m + 1) / 2;
    __syncthreads();
  }
  if (wave != 0) return;
  const int n = s.cnt[0];
  const uint32_t flags = s.flags;
  const uint64_t v = lane < n ? lists[lane] : 0ull;
  if (INLINE) {
    if (flags & kFlagBadHistory) {
      if (lane == 0) a.out_ids[row] = ARBOR_ID_BAD_HISTORY;
    } else if (flags & kFlagInvalid) {
      if (lane == 0) a.out_ids[row] = ARBOR_ID_INVALID;
    } else if (n == 0) {
      if (lane == 0) a.out_ids[row] = ARBOR_ID_EMPTY;
    } else {
      finish_list(a, row, v, n);
    }
  } else {
    const size_t slot = (size_t)row * (size_t)a.S + (size_t)chunk;
    if (lane < n) a.cand[slot * kChunkSlot + lane] = v;
    if (lane == 0) {
      a.hdr[slot * 2 + 0] = (uint32_t)n;
      a.hdr[slot * 2 + 1] = flags;
    }
  }
}

// Finishes top-k rows that were split into chunks: one wave per row merges the chunks'
// lists and draws.
__global__ void __launch_bounds__(256) topk_finish_kernel(Args a) {
  const int lane = lane_id();
  const int row = blockIdx.x * 4 + (int)threadIdx.x / kWave;
  if (row >= a.B) return;
  uint32_t flags = 0u;
  uint64_t best = 0ull;
  for (int c0 = 0; c0 < a.S; c0 += 8) {
    uint64_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + j;
      v[j] = 0ull;
      if (c < a.S) {
        const size_t slot = (size_t)row * (size_t)a.S + (size_t)c;
        const int n = (int)a.hdr[slot * 2 + 0];
        flags |= a.hdr[slot * 2 + 1];
        if (lane < n) v[j] = a.cand[slot * kChunkSlot + lane];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c0 + j < a.S) best = list_merge(best, v[j]);
  }
  const int n = min(a.top_k, list_count(best));
  if (flags & kFlagBadHistory) {
    if (lane == 0) a.out_ids[row] = ARBOR_ID_BAD_HISTORY;
  } else if (flags & kFlagInvalid) {
    if (lane == 0) a.out_ids[row] = ARBOR_ID_INVALID;
  } else if (n == 0) {
    if (lane == 0) a.out_ids[row] = ARBOR_ID_EMPTY;
  } else {
    finish_list(a, row, best, n);
  }
}

// Finishes rows that were split into chunks: merges the chunks' lists, adds the history
// ids and draws. One workgroup per row.
template <int DT, bool MODE_K>
__global__ void __launch_bounds__(kBlock) finish_kernel(Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  Lds L(smem);
  __shared__ FinishShared s;
  const int t = threadIdx.x, row = blockIdx.x;
  if (t == 0) s.flags = 0u;
  __syncthreads();
  if (t < a.S) {
    const size_t slot = (size_t)row * (size_t)a.S + (size_t)t;
    s.cnt[t] = (int)a.hdr[slot * 2 + 0];
    atomicOr(&s.flags, a.hdr[slot * 2 + 1]);
  }
  __syncthreads();
  if (t == 0) {
    int o = 0;
    for (int c = 0; c < a.S; ++c) {
      s.off[c] = o;
      o += s.cnt[c];
    }
    s.ints[0] = o;
  }
  __syncthreads();
  // load every list at once: each thread fetches up to 4 entries before storing any
  constexpr int R = 4;
  const int total = s.ints[0];
  uint64_t v[R];
  int at[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int f = t + r * kBlock;
    at[r] = -1;
    if (f < total) {
      int c = 0;
      while (f >= s.off[c] + s.cnt[c]) ++c;
      v[r] = a.cand[((size_t)row * (size_t)a.S + (size_t)c) * kChunkSlot + (size_t)(f - s.off[c])];
      at[r] = f;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (at[r] >= 0) L.lists[at[r]] = v[r];
  __syncthreads();
  finish_row<kBlock, DT, MODE_K>(a, row, L.lists, a.S, s.flags, L, s);
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
  bool mode_k;      // stream path: top-k (else: min-p band)
  bool inline_fin;  // stream path: one chunk per row, finished in the same workgroup
  int k;            // effective top-k (0 = off)
  int S, chunk_len;
  int hash_bits, bitmap_words;
  size_t lds_stream, lds_finish, lds_solver;
  // workspace layout (byte offsets)
  size_t off_hdr, off_cand, off_zbuf, total;
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
  if (!(p->repetition_penalty > 0.0f) || !std::isfinite(p->repetition_penalty) ||
      !std::isfinite(p->frequency_penalty) || !std::isfinite(p->presence_penalty))
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

// Compute units of the current device (cached per device; 256 on MI355X).
int device_cus() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

Plan make_plan(const arbor_sampling_params* p, int cus) {
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
  pl.S = 1;
  if (pl.path == Path::Stream) {
    // one 1024-thread workgroup per compute unit: split rows only when the batch is
    // smaller than the chip, and never below 8K ids per chunk
    int S = B < cus ? cus / B : 1;
    const int by_len = (V + 8191) / 8192;
    if (S > by_len) S = by_len;
    const int slots = pl.mode_k ? arbor::kWaves * arbor::kWaveCap / 2 / pl.k
                                : arbor::kWaves * arbor::kWaveCap / 2 / arbor::kChunkSlot;
    if (S > slots) S = slots;
    if (S > arbor::kMaxChunks) S = arbor::kMaxChunks;
    const int by_bitmap = (V + arbor::kMaxChunkLen - 1) / arbor::kMaxChunkLen;
    if (S < by_bitmap) S = by_bitmap;
    if (S < 1) S = 1;
    const int len = (int)align_up((size_t)((V + S - 1) / S), 512);
    S = (V + len - 1) / len;
    pl.S = S;
    pl.chunk_len = len;
    pl.inline_fin = S == 1;
    pl.bitmap_words = p->hist_len > 0 ? len / 32 : 0;
    pl.lds_stream = pl.mode_k ? arbor::topk_lds_bytes(p->hist_len > 0 ? (1 << hb) : 0, pl.bitmap_words)
                              : arbor::lds_total(pl.bitmap_words);
    pl.lds_finish = arbor::lds_total(0);
  }
  pl.lds_solver = sizeof(uint32_t) * (size_t)(1 << hb);
  size_t off = 0;
  pl.off_hdr = off;
  off = align_up(off + sizeof(uint32_t) * 2 * (size_t)B * (size_t)pl.S, 256);
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

template <int DT, bool PEN, bool MASK, bool MODE_K>
int launch_stream4(bool inl, dim3 grid, size_t lds, hipStream_t st, const arbor::Args& a) {
  const dim3 block(arbor::kBlock);
  if (inl) return launch(arbor::stream_kernel<DT, PEN, MASK, MODE_K, true>, grid, block, lds, st, a);
  return launch(arbor::stream_kernel<DT, PEN, MASK, MODE_K, false>, grid, block, lds, st, a);
}

// the LDS-buffer streaming kernel serves the min-p band; top-k goes to topk_kernel
template <int DT, bool PEN, bool MASK>
int launch_stream3(bool mode_k, bool inl, dim3 grid, size_t lds, hipStream_t st, const arbor::Args& a) {
  (void)mode_k;
  return launch_stream4<DT, PEN, MASK, false>(inl, grid, lds, st, a);
}

template <int DT, bool PEN, bool MASK>
int launch_topk3(const Plan& pl, hipStream_t st, const arbor::Args& a) {
  const dim3 grid((unsigned)(a.B * pl.S)), block(arbor::kBlock);
  int r = pl.inline_fin ? launch(arbor::topk_kernel<DT, PEN, MASK, true>, grid, block, pl.lds_stream, st, a)
                        : launch(arbor::topk_kernel<DT, PEN, MASK, false>, grid, block, pl.lds_stream, st, a);
  if (r != ARBOR_OK || pl.inline_fin) return r;
  return launch(arbor::topk_finish_kernel, dim3((unsigned)((a.B + 3) / 4)), dim3(256), 0, st, a);
}

template <int DT>
int launch_topk(const Plan& pl, bool pen, bool mask, hipStream_t st, const arbor::Args& a) {
  if (pen) return mask ? launch_topk3<DT, true, true>(pl, st, a) : launch_topk3<DT, true, false>(pl, st, a);
  return mask ? launch_topk3<DT, false, true>(pl, st, a) : launch_topk3<DT, false, false>(pl, st, a);
}

template <int DT>
int launch_stream(const Plan& pl, bool pen, bool mask, hipStream_t st, const arbor::Args& a) {
  if (pl.mode_k) return launch_topk<DT>(pl, pen, mask, st, a);
  const dim3 grid((unsigned)(a.B * pl.S));
  int r;
  if (pen)
    r = mask ? launch_stream3<DT, true, true>(pl.mode_k, pl.inline_fin, grid, pl.lds_stream, st, a)
             : launch_stream3<DT, true, false>(pl.mode_k, pl.inline_fin, grid, pl.lds_stream, st, a);
  else
    r = mask ? launch_stream3<DT, false, true>(pl.mode_k, pl.inline_fin, grid, pl.lds_stream, st, a)
             : launch_stream3<DT, false, false>(pl.mode_k, pl.inline_fin, grid, pl.lds_stream, st, a);
  if (r != ARBOR_OK || pl.inline_fin) return r;
  const dim3 fgrid((unsigned)a.B), block(arbor::kBlock);
  if (pl.mode_k) return launch(arbor::finish_kernel<DT, true>, fgrid, block, pl.lds_finish, st, a);
  return launch(arbor::finish_kernel<DT, false>, fgrid, block, pl.lds_finish, st, a);
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
  return make_plan(p, device_cus()).total;
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
  const Plan pl = make_plan(p, device_cus());
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
  a.hash_bits = pl.hash_bits;
  a.bitmap_words = pl.bitmap_words;
  const size_t esz = p->dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
  a.aligned = ((uintptr_t)logits % 16 == 0) && (((size_t)p->ld_logits * esz) % 16 == 0);
  a.write_probs = probs ? 1 : 0;
  char* ws = static_cast<char*>(workspace);
  a.hdr = reinterpret_cast<uint32_t*>(ws + pl.off_hdr);
  a.cand = reinterpret_cast<uint64_t*>(ws + pl.off_cand);
  a.zbuf = reinterpret_cast<float*>(ws + pl.off_zbuf);
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (pl.path == Path::Solver) {
    const dim3 grid(p->batch), block(arbor::kBlock);
    if (p->dtype == ARBOR_DTYPE_BF16)
      return launch(arbor::solver_kernel<ARBOR_DTYPE_BF16>, grid, block, pl.lds_solver, s, a);
    return launch(arbor::solver_kernel<ARBOR_DTYPE_F32>, grid, block, pl.lds_solver, s, a);
  }
  const bool pen = p->hist_len > 0, mask = allow_mask != nullptr;
  if (p->dtype == ARBOR_DTYPE_BF16) return launch_stream<ARBOR_DTYPE_BF16>(pl, pen, mask, s, a);
  return launch_stream<ARBOR_DTYPE_F32>(pl, pen, mask, s, a);
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
