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
      thr = fmaxf(thr, key_value(lane_get(key, a.top_k - 1)));
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
    return lane_get(b, 0);
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
// Streaming top-k (1 <= k <= 64)
//
//  A. Threshold: the k-th best of the 1024 lane maxima of every wave's first two batches
//     is a lower bound T0 of the row's k-th best (the k-th best of a subset never exceeds
//     the k-th best of the whole); it is found with one 2048-bin histogram over the keys'
//     observed range, taking the lower edge of the bin that holds the k-th maximum.
//  B. Stream: everything >= the wave's threshold (T0, raised by an exact wave radix
//     select if the wave's buffer fills) is appended to a per-wave LDS buffer.
//  C. Select: the wave buffers and the penalised history ids >= T0 form the union; a block
//     radix select finds its k-th best; one wave sorts the k survivors and draws (fp64).
// ---------------------------------------------------------------------------------------
constexpr int kTopkWaveCap = 256;   // candidates one wave buffers
constexpr int kUnionCap = 4096;     // candidates the row's selection runs over
constexpr int kSampleBins = 2048;   // histogram bins of the threshold sample

struct TopkShared {
  int next_batch;
  uint32_t flags;
  int n_union;
  int n_top;
  float t0;
  int dsel;
  uint32_t above, csel;
  int cnt[kWaves];
  int off[kWaves + 1];
  uint32_t red[kWaves];
  uint64_t red64[kWaves];
};

// Dynamic LDS of topk_kernel (bytes): wave buffers | histograms | chunk bitmap |
// history candidates | history table (later the union).
struct TopkLds {
  uint64_t* wb;      // [kWaves * kTopkWaveCap]
  uint32_t* hist;    // [kWaves * 256] (also the 2048-bin sample histogram; solver scratch)
  uint32_t* bitmap;  // [bitmap_words]
  uint64_t* hc;      // [hist_len] penalised history candidates
  uint32_t* htab;    // [1 << hash_bits], then overlaid by
  uint64_t* uni;     // [kUnionCap]
  __host__ __device__ static size_t bytes(int bitmap_words, int hist_len, int hash_slots) {
    const size_t tail = sizeof(uint32_t) * (size_t)hash_slots > sizeof(uint64_t) * kUnionCap
                            ? sizeof(uint32_t) * (size_t)hash_slots
                            : sizeof(uint64_t) * kUnionCap;
    return sizeof(uint64_t) * kWaves * kTopkWaveCap + sizeof(uint32_t) * kWaves * 256 +
           (sizeof(uint32_t) * (size_t)bitmap_words + 7) / 8 * 8 + sizeof(uint64_t) * (size_t)hist_len + tail;
  }
  __device__ TopkLds(unsigned char* base, int bitmap_words, int hist_len) {
    wb = reinterpret_cast<uint64_t*>(base);
    hist = reinterpret_cast<uint32_t*>(wb + kWaves * kTopkWaveCap);
    bitmap = hist + kWaves * 256;
    hc = reinterpret_cast<uint64_t*>(reinterpret_cast<unsigned char*>(bitmap) +
                                     ((size_t)bitmap_words * sizeof(uint32_t) + 7) / 8 * 8);
    htab = reinterpret_cast<uint32_t*>(hc + hist_len);
    uni = reinterpret_cast<uint64_t*>(htab);
  }
};

// Composite T such that exactly min(k, n) of the n distinct composites u[0, n) are >= T:
// MSB-first radix select, 8-bit digits below the highest bit in which they differ.
template <int BLOCK>
__device__ uint64_t block_select_kth(const uint64_t* u, int n, int k, uint32_t* hist, TopkShared& s) {
  const int t = threadIdx.x;
  if (n <= k) return 0ull;
  uint64_t lo = ~0ull, hi = 0ull;
  for (int i = t; i < n; i += BLOCK) {
    lo = u[i] < lo ? u[i] : lo;
    hi = u[i] > hi ? u[i] : hi;
  }
  lo = block_reduce_min<BLOCK, uint64_t>(lo, s.red64);
  hi = block_reduce_max<BLOCK, uint64_t>(hi, s.red64);
  const int hb = 63 - __clzll(hi ^ lo);
  int shift = hb >= 7 ? hb - 7 : 0;
  uint64_t pmask = hb >= 63 ? 0ull : (~0ull << (hb + 1));
  uint64_t prefix = hi & pmask;
  uint32_t need = (uint32_t)k;
  for (;;) {
    if (t < 256) hist[t] = 0u;
    __syncthreads();
    for (int i = t; i < n; i += BLOCK) {
      const uint64_t c = u[i];
      if ((c & pmask) == prefix) atomicAdd(&hist[(uint32_t)(c >> shift) & 255u], 1u);
    }
    __syncthreads();
    const uint32_t cnt = t < 256 ? hist[255 - t] : 0u;  // descending digits
    uint32_t tot;
    const uint32_t ex = block_scan_excl<BLOCK, uint32_t>(cnt, s.red, &tot);
    if (t < 256 && ex < need && ex + cnt >= need) {
      s.dsel = 255 - t;
      s.above = ex;
      s.csel = cnt;
    }
    __syncthreads();
    const int dsel = s.dsel;
    const uint32_t above = s.above, csel = s.csel;
    __syncthreads();
    need -= above;
    prefix = (prefix & ~(255ull << shift)) | ((uint64_t)dsel << shift);
    pmask |= 255ull << shift;
    if (need == csel || shift == 0) return prefix;
    shift = shift >= 8 ? shift - 8 : 0;
  }
}

template <int DT, bool PEN, bool MASK, bool INLINE, bool ALIGNED>
__global__ void __launch_bounds__(kBlock) topk_kernel(Args a) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int U = Elem<DT>::kUnroll;
  constexpr int NQ = VEC * U;                       // elements per lane per batch
  constexpr int kBatch = U * kWave;                 // units per batch
  constexpr int HR = (1 << kMaxHashBits) / kBlock;  // history-table slots per thread
  constexpr int HIDR = (ARBOR_HISTORY_MAX + kBlock - 1) / kBlock;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ TopkShared s;
  const bool own_hist = PEN && (blockIdx.x % a.S) == 0;  // this workgroup evaluates the row's history
  TopkLds L(smem, PEN ? a.bitmap_words : 0, own_hist ? a.H : 0);

  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  const int row = blockIdx.x / a.S, chunk = blockIdx.x % a.S;
  const int c0 = chunk * a.chunk_len;
  const int c1 = min(a.V, c0 + a.chunk_len);
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = MASK ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const int n_units = (c1 - c0 + VEC - 1) / VEC;
  const int n_batches = (n_units + kBatch - 1) / kBatch;
  const int k = a.top_k;

  // Aligned rows: every lane issues exactly one 16-byte load per unit (a unit past the
  // chunk reloads the chunk's last unit and is ignored), so the compiler can count the
  // loads in flight and the next batch overlaps the current one.
  struct Batch {
    uint32_t w[U][4];  // raw 16-byte units
    uint32_t mw[U];
  };
  auto load = [&](int bi, Batch& bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int unit = bi * kBatch + u * kWave + lane;
      if (ALIGNED) {
        const int e0 = c0 + (unit < n_units ? unit : n_units - 1) * VEC;
        typedef unsigned int u4 __attribute__((ext_vector_type(4)));
        const u4 v = __builtin_nontemporal_load(
            reinterpret_cast<const u4*>(static_cast<const char*>(xrow) + (size_t)e0 * Elem<DT>::kBytes));
        bt.w[u][0] = v.x;
        bt.w[u][1] = v.y;
        bt.w[u][2] = v.z;
        bt.w[u][3] = v.w;
        if (MASK) bt.mw[u] = mrow[e0 >> 5];
      } else {
        const int e0 = c0 + unit * VEC;
        load_raw<DT>(xrow, e0, c1, false, bt.w[u]);
        if (MASK) bt.mw[u] = e0 < c1 ? mrow[e0 >> 5] : 0u;
      }
    }
  };
  // tempered logit of slot q of batch b; history ids (scored separately, penalised),
  // masked ids and units past the chunk read as -inf; NaN / +inf read as -inf (flagged
  // by `process`)
  auto zof = [&](int b, const Batch& bt, int q) -> float {
    const int u = q / VEC, j = q % VEC;
    const int unit = b * kBatch + u * kWave + lane;
    const int e0 = c0 + unit * VEC;
    if (unit >= n_units) return -INFINITY;
    float v = unpack_unit<DT>(bt.w[u], j) * a.inv_t;
    if (PEN && ((L.bitmap[(e0 - c0) >> 5] >> (((e0 - c0) & 31) + j)) & 1u)) v = -INFINITY;
    if (MASK && !((bt.mw[u] >> ((e0 & 31) + j)) & 1u)) v = -INFINITY;
    return is_invalid(v) ? -INFINITY : v;
  };

  // two batches per wave are in flight while the workgroup sets up
  Batch ba, bb;
  int ia = wave, ib = wave + kWaves;
  load(ia, ba);
  load(ib, bb);

  int32_t hid[HIDR];
  if (PEN) {
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
#pragma unroll
    for (int r = 0; r < HIDR; ++r) {
      const int j = t + r * kBlock;
      hid[r] = j < a.H ? h[j] : -1;
    }
  }
  if (t == 0) {
    s.next_batch = 2 * kWaves;
    s.flags = 0u;
    s.n_union = 0;
    s.n_top = 0;
  }
  if (PEN) {
    for (int i = t; i < a.bitmap_words; i += kBlock) L.bitmap[i] = 0u;
    if (own_hist)
      for (int i = t; i < (1 << a.hash_bits); i += kBlock) L.htab[i] = kEmptySlot;
  }
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = c0 + t; i < c1; i += kBlock) prow[i] = 0.0f;
  }
  __syncthreads();
  if (PEN) {
    bool bad = false;
#pragma unroll
    for (int r = 0; r < HIDR; ++r) {
      const int32_t id = hid[r];
      if (id >= a.V) {
        bad = true;
      } else if (id >= 0) {
        if (id >= c0 && id < c1) atomicOr(&L.bitmap[(id - c0) >> 5], 1u << ((id - c0) & 31));
        if (own_hist) hist_insert(L.htab, (uint32_t)a.hash_bits, (uint32_t)id);
      }
    }
    if (bad) atomicOr(&s.flags, kFlagBadHistory);
  }
  __syncthreads();

  // ---- the row's distinct history ids, penalised, into hc[] (every thread: HR slots) ----
  bool bad = false;
  if (own_hist) {
    const int P = 1 << a.hash_bits;
    int idq[HR];
    uint32_t cq[HR], mq[HR];
    float xq[HR];
#pragma unroll
    for (int r = 0; r < HR; ++r) {
      const int slot = t + r * kBlock;
      const uint32_t e = slot < P ? L.htab[slot] : kEmptySlot;
      idq[r] = e != kEmptySlot ? (int)(e >> 12) : -1;
      cq[r] = (e & 4095u) + 1u;
      xq[r] = idq[r] >= 0 ? Elem<DT>::one(xrow, idq[r]) : 0.0f;
      mq[r] = (MASK && idq[r] >= 0) ? mrow[idq[r] >> 5] : ~0u;
    }
#pragma unroll
    for (int r = 0; r < HR; ++r) {
      if (idq[r] < 0) continue;
      float z = penalize(xq[r] * a.inv_t + 0.0f, cq[r], a.pen);
      if (!((mq[r] >> (idq[r] & 31)) & 1u)) z = -INFINITY;
      if (is_invalid(z)) {
        bad = true;
      } else if (z != -INFINITY) {
        L.hc[atomicAdd(&s.n_top, 1)] = composite(z, idq[r]);  // n_top counts hc[] here
      }
    }
  }

  // ---- A. threshold from the lane maxima of the first two batches ----
  {
    float lm = -INFINITY;
#pragma unroll
    for (int q = 0; q < NQ; ++q) lm = fmaxf(lm, zof(ia, ba, q));
#pragma unroll
    for (int q = 0; q < NQ; ++q) lm = fmaxf(lm, zof(ib, bb, q));
    const uint32_t key = order_key(lm);
    const uint32_t kmin = block_reduce_min<kBlock, uint32_t>(key, s.red);
    const uint32_t kmax = block_reduce_max<kBlock, uint32_t>(key, s.red);
    const uint32_t span = kmax - kmin;
    const int sh = span == 0u ? 0 : max(0, 32 - __clz(span) - 11);
    for (int i = t; i < kSampleBins; i += kBlock) L.hist[i] = 0u;
    __syncthreads();
    atomicAdd(&L.hist[(key - kmin) >> sh], 1u);
    __syncthreads();
    // bins in descending order, two per thread
    const uint32_t h0 = L.hist[kSampleBins - 1 - 2 * t], h1 = L.hist[kSampleBins - 2 - 2 * t];
    uint32_t tot;
    const uint32_t ex = block_scan_excl<kBlock, uint32_t>(h0 + h1, s.red, &tot);
    if (t == 0) s.t0 = -FLT_MAX;
    __syncthreads();
    int bsel = -1;
    if (ex < (uint32_t)k && ex + h0 >= (uint32_t)k)
      bsel = kSampleBins - 1 - 2 * t;
    else if (ex + h0 < (uint32_t)k && ex + h0 + h1 >= (uint32_t)k)
      bsel = kSampleBins - 2 - 2 * t;
    if (bsel >= 0) {
      const float tz = key_value(kmin + ((uint32_t)bsel << sh));
      s.t0 = tz > -FLT_MAX ? tz : -FLT_MAX;
    }
    __syncthreads();
  }
  const float t0 = s.t0;

  // ---- B. stream: batches from an LDS counter, two in flight per wave ----
  uint64_t* buf = L.wb + wave * kTopkWaveCap;
  uint32_t* rh = L.hist + wave * 256;
  int wc = 0;
  float thr = t0;  // append z >= thr
  bool ovf = false;
  auto grab = [&]() -> int {
    int b = 0;
    if (lane == 0) b = atomicAdd(&s.next_batch, 1);
    return lane_get(b, 0);
  };
  __syncthreads();  // the sample histogram is no longer read: wave radix histograms may reuse it
  auto process = [&](int b, const Batch& bt) {
    uint32_t pend = 0u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int unit = b * kBatch + u * kWave + lane;
      const int e0 = c0 + unit * VEC;
      const bool valid = unit < n_units;
      const uint32_t mb = MASK ? bt.mw[u] >> (e0 & 31) : ~0u;
      const uint32_t pb = PEN && valid ? L.bitmap[(e0 - c0) >> 5] >> ((e0 - c0) & 31) : 0u;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float v = unpack_unit<DT>(bt.w[u], j) * a.inv_t;
        const bool skip = !valid || (PEN && ((pb >> j) & 1u)) || (MASK && !((mb >> j) & 1u));
        bad |= !skip && is_invalid(v);
        if (!skip && v >= thr && !is_invalid(v)) pend |= 1u << (u * VEC + j);
      }
    }
    if (!__ballot(pend != 0u) || ovf) return;
    int cnt = wave_sum((int)__popc(pend));
    if (wc + cnt > kTopkWaveCap) {
      if (wc > k) thr = fmaxf(thr, wave_keep_topk<kTopkWaveCap>(buf, wc, k, rh));
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        if (((pend >> q) & 1u) && !(zof(b, bt, q) >= thr)) pend &= ~(1u << q);
      cnt = wave_sum((int)__popc(pend));
      if (wc + cnt > kTopkWaveCap) {
        // a batch denser than the buffer: 64 candidates at a time, an exact prune between
#pragma unroll 1
        for (int q = 0; q < NQ; ++q) {
          float v = -INFINITY;
#pragma unroll
          for (int qq = 0; qq < NQ; ++qq)
            if (qq == q && ((pend >> qq) & 1u)) v = zof(b, bt, qq);
          if (!__ballot(v >= thr)) continue;
          if (wc + kWave > kTopkWaveCap) {
            thr = fmaxf(thr, wave_keep_topk<kTopkWaveCap>(buf, wc, k, rh));
            if (wc + kWave > kTopkWaveCap) {
              ovf = true;  // unreachable for k <= 64: the row would go to the row solver
              return;
            }
          }
          const bool take = v >= thr;
          const uint64_t bal = __ballot(take);
          if (take) buf[wc + lanes_below(bal)] =
              composite(v + 0.0f, c0 + (b * kBatch + (q / VEC) * kWave + lane) * VEC + (q % VEC));
          wc += __popcll(bal);
        }
        return;
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const bool tk = (pend >> q) & 1u;
      const uint64_t bal = __ballot(tk);
      if (bal) {
        if (tk)
          buf[wc + lanes_below(bal)] =
              composite(zof(b, bt, q) + 0.0f, c0 + (b * kBatch + (q / VEC) * kWave + lane) * VEC + (q % VEC));
        wc += __popcll(bal);
      }
    }
  };
  for (;;) {
    if (ia >= n_batches) break;
    process(ia, ba);
    ia = grab();
    load(ia, ba);
    if (ib >= n_batches) break;
    process(ib, bb);
    ib = grab();
    load(ib, bb);
  }
  if (lane == 0) s.cnt[wave] = wc;
  if (__ballot(bad) && lane == 0) atomicOr(&s.flags, kFlagInvalid);
  if (__ballot(ovf) && lane == 0) atomicOr(&s.flags, kFlagOverflow);
  __syncthreads();

  // ---- C. union of the wave buffers and the history candidates >= t0; exact top-k ----
  if (t == 0) {
    int o = 0;
    for (int w = 0; w < kWaves; ++w) {
      s.off[w] = o;
      o += s.cnt[w];
    }
    s.off[kWaves] = o;
    if (o > kUnionCap) s.flags |= kFlagOverflow;
    s.n_union = o > kUnionCap ? 0 : o;
  }
  __syncthreads();
  const int n_hc = own_hist ? s.n_top : 0;
  if (!(s.flags & kFlagOverflow)) {
    for (int i = lane; i < s.cnt[wave]; i += kWave) L.uni[s.off[wave] + i] = buf[i];
    for (int i = t; i < n_hc; i += kBlock) {
      const uint64_t c = L.hc[i];
      if (composite_z(c) >= t0) {
        const int pos = atomicAdd(&s.n_union, 1);
        if (pos < kUnionCap)
          L.uni[pos] = c;
        else
          atomicOr(&s.flags, kFlagOverflow);
      }
    }
  }
  __syncthreads();
  const uint32_t flags = s.flags;
  if ((flags & kFlagOverflow) && !(flags & (kFlagBadHistory | kFlagInvalid))) {
    if (INLINE) {
      solve_row<kBlock, DT>(a, row, L.htab, *reinterpret_cast<SolverShared*>(L.hist));
    } else if (t == 0) {
      const size_t slot = (size_t)row * (size_t)a.S + (size_t)chunk;
      a.hdr[slot * 2 + 0] = 0u;
      a.hdr[slot * 2 + 1] = flags;
    }
    return;
  }
  const int nu = s.n_union;
  const uint64_t T = block_select_kth<kBlock>(L.uni, nu, k, L.hist, s);
  if (t == 0) s.n_top = 0;
  __syncthreads();
  for (int i = t; i < nu; i += kBlock)
    if (L.uni[i] >= T) L.wb[atomicAdd(&s.n_top, 1)] = L.uni[i];  // the k best, unordered
  __syncthreads();
  if (wave != 0) return;
  const int n = s.n_top;
  uint64_t v = lane < n ? L.wb[lane] : 0ull;
  v = wave_sort64_desc(v);
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

// Finishes top-k rows that were split into chunks: wave 0 of a workgroup per row merges
// the chunks' lists and draws; a row with an overflowed chunk is solved exactly.
template <int DT>
__global__ void __launch_bounds__(kBlock) topk_finish_kernel(Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SolverShared ssh;
  __shared__ uint32_t s_flags;
  const int lane = lane_id(), row = blockIdx.x;
  if (threadIdx.x == 0) {
    uint32_t f = 0u;
    for (int c = 0; c < a.S; ++c) f |= a.hdr[((size_t)row * (size_t)a.S + (size_t)c) * 2 + 1];
    s_flags = f;
  }
  __syncthreads();
  const uint32_t flags = s_flags;
  if ((flags & kFlagOverflow) && !(flags & (kFlagBadHistory | kFlagInvalid))) {
    solve_row<kBlock, DT>(a, row, reinterpret_cast<uint32_t*>(smem), ssh);
    return;
  }
  if (threadIdx.x >= kWave) return;
  uint64_t best = 0ull;
  for (int cb = 0; cb < a.S; cb += 8) {
    uint64_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = cb + j;
      v[j] = 0ull;
      if (c < a.S) {
        const size_t slot = (size_t)row * (size_t)a.S + (size_t)c;
        const int n = (int)a.hdr[slot * 2 + 0];
        if (lane < n) v[j] = a.cand[slot * kChunkSlot + lane];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (cb + j < a.S) best = list_merge(best, v[j]);
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
    pl.lds_stream = pl.mode_k ? arbor::TopkLds::bytes(pl.bitmap_words, p->hist_len, p->hist_len > 0 ? (1 << hb) : 0)
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

template <int DT, bool PEN, bool MASK, bool ALIGNED>
int launch_topk4(const Plan& pl, hipStream_t st, const arbor::Args& a) {
  const dim3 grid((unsigned)(a.B * pl.S)), block(arbor::kBlock);
  int r = pl.inline_fin
              ? launch(arbor::topk_kernel<DT, PEN, MASK, true, ALIGNED>, grid, block, pl.lds_stream, st, a)
              : launch(arbor::topk_kernel<DT, PEN, MASK, false, ALIGNED>, grid, block, pl.lds_stream, st, a);
  if (r != ARBOR_OK || pl.inline_fin) return r;
  return launch(arbor::topk_finish_kernel<DT>, dim3((unsigned)a.B), block, pl.lds_solver, st, a);
}

template <int DT, bool PEN, bool MASK>
int launch_topk3(const Plan& pl, hipStream_t st, const arbor::Args& a) {
  // whole 16-byte units only: aligned rows whose length is a multiple of the unit
  if (a.aligned && a.V % arbor::Elem<DT>::kVec == 0) return launch_topk4<DT, PEN, MASK, true>(pl, st, a);
  return launch_topk4<DT, PEN, MASK, false>(pl, st, a);
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
