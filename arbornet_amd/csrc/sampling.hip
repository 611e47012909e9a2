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
#include <mutex>

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
// Streaming top-k (1 <= k <= 64): one workgroup per row, or per chunk of a row.
//
//  Set-up: the row's history ids are loaded ahead of the logits and fill an LDS bitmap of
//     the chunk's history ids and an id -> count table while the first two batches of
//     every wave are in flight.
//  A. Threshold: T0 is a lower bound of the k-th largest of the 1024 lane maxima of every
//     wave's first two batches (the k-th largest of a subset never exceeds the k-th
//     largest of the whole): a histogram of the order keys' top 10 bits, then of the next
//     10 bits inside the bin that holds the k-th; every wave reads the bins itself.
//  B. Stream: everything >= the wave's threshold is appended to a per-wave LDS buffer; a
//     full buffer is cut to its exact k best (wave radix select), raising the threshold.
//     When no penalty can raise a logit (repetition >= 1, frequency and presence >= 0)
//     history ids stream past like the others and only those whose raw z passes are
//     penalised; otherwise they are skipped and scored once at set-up.
//  C. Finish: each wave sorts its k best (bitonic network over DPP), a tree of bitonic
//     merges (four barriers) leaves the chunk's k best in wave 0, which draws in fp64 or
//     publishes them for the row's finish kernel.
// ---------------------------------------------------------------------------------------
constexpr int kTopkWaveCap = 256;  // candidates one wave buffers
constexpr int kBinBits = 10;       // threshold histograms: 2 x 10 bits of the order key
constexpr int kBins = 1 << kBinBits;
#ifndef TOPK_UNROLL_F32
#define TOPK_UNROLL_F32 3
#endif

// Counts of 10-bit key digits with a 64-bin summary (16 bins each), so that the bin of
// the need-th largest entry is found with two wave scans.
struct KeyHist {
  uint32_t fine[kBins];
  uint32_t coarse[kBins / 16];
};
__device__ __forceinline__ void key_hist_add(KeyHist& h, uint32_t bin) {
  atomicAdd(&h.fine[bin], 1u);
  atomicAdd(&h.coarse[bin >> 4], 1u);
}
// Bin holding the need-th largest entry (1 <= need <= total), counted from the top bin
// down; *above = entries in higher bins. Every lane of the wave gets the result.
__device__ __forceinline__ int key_hist_kth(const KeyHist& h, uint32_t need, uint32_t* above) {
  static_assert(kBins / 16 == kWave, "one summary bin per lane");
  const int lane = lane_id();
  const uint32_t cc = h.coarse[kWave - 1 - lane];  // lane l: l-th highest summary bin
  const uint32_t ci = wave_scan_incl(cc);
  const uint64_t hit = __ballot(ci >= need);
  if (!hit) {
    *above = lane_get(ci, kWave - 1);
    return 0;
  }
  const int lc = __ffsll((long long)hit) - 1;
  const uint32_t base = lane_get(ci - cc, lc);
  const int cbin = kWave - 1 - lc;
  const uint32_t cf = lane < 16 ? h.fine[cbin * 16 + 15 - lane] : 0u;
  const uint32_t fi = wave_scan_incl(cf);
  const int lf = __ffsll((long long)__ballot(lane < 16 && base + fi >= need)) - 1;
  *above = base + lane_get(fi - cf, lf);
  return cbin * 16 + 15 - lf;
}

// 16-byte loads per lane per batch of the streaming top-k kernel (two batches in flight)
template <int DT>
struct TopkUnroll {
  static constexpr int value = DT == ARBOR_DTYPE_F32 ? TOPK_UNROLL_F32 : 2;
};

struct TopkShared {
  int next_batch;
  uint32_t flags;
  int n_sel;  // entries at or above the final selection's bin edge
};

// Dynamic LDS of topk_kernel (bytes): wave buffers | radix histograms | threshold
// histograms | chunk bitmap | history candidates | history table.
struct TopkLds {
  uint64_t* wb;      // [kWaves * kTopkWaveCap]; at the end the waves' sorted lists
  uint32_t* hist;    // [kWaves * 256] wave radix histograms (row solver scratch on fallback)
  KeyHist* kh;       // [4] threshold sample (two levels), final selection (two levels)
  uint64_t* sel;     // [kWave] the chunk's k best, unordered
  uint64_t* side;    // [kWaves * kWave] history ids whose raw z passed (penalised at the end)
  uint32_t* bitmap;  // [bitmap_words]
  uint32_t* htab;    // [hash_slots]
  __host__ __device__ static size_t bytes(int bitmap_words, int hash_slots) {
    return sizeof(uint64_t) * kWaves * (kTopkWaveCap + kWave) + sizeof(uint32_t) * kWaves * 256 +
           sizeof(KeyHist) * 4 + sizeof(uint64_t) * kWave + sizeof(uint32_t) * (size_t)bitmap_words +
           sizeof(uint32_t) * (size_t)hash_slots;
  }
  __device__ TopkLds(unsigned char* base, int bitmap_words) {
    wb = reinterpret_cast<uint64_t*>(base);
    side = wb + kWaves * kTopkWaveCap;
    hist = reinterpret_cast<uint32_t*>(side + kWaves * kWave);
    kh = reinterpret_cast<KeyHist*>(hist + kWaves * 256);
    sel = reinterpret_cast<uint64_t*>(kh + 4);
    bitmap = reinterpret_cast<uint32_t*>(sel + kWave);
    htab = bitmap + bitmap_words;
  }
};

template <int DT, bool PEN, bool MASK, bool INLINE, bool ALIGNED>
__global__ void __launch_bounds__(kBlock) topk_kernel(Args a) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int U = TopkUnroll<DT>::value;
  constexpr int NQ = VEC * U;                       // elements per lane per batch
  constexpr int kBatch = U * kWave;                 // units per batch
  constexpr int HIDR = (ARBOR_HISTORY_MAX + kBlock - 1) / kBlock;
  static_assert(sizeof(SolverShared) <= sizeof(uint32_t) * kWaves * 256, "solver scratch fits the radix histograms");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ TopkShared s;
  // history ids stream past and are penalised inline, or are scored here at set-up by
  // the first chunk of the row
  const bool hist_inline = PEN && a.pen_mono;
  const bool own_hist = PEN && !hist_inline && (blockIdx.x % a.S) == 0;
  TopkLds L(smem, PEN ? a.bitmap_words : 0);

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
  // tempered logit of slot q of batch b for the threshold sample: history ids, masked ids,
  // units past the chunk and NaN / +inf read as -inf (the sample leaves them out)
  auto zsample = [&](int b, const Batch& bt, int q) -> float {
    const int u = q / VEC, j = q % VEC;
    const int unit = b * kBatch + u * kWave + lane;
    const int e0 = c0 + unit * VEC;
    if (unit >= n_units) return -INFINITY;
    float v = unpack_unit<DT>(bt.w[u], j) * a.inv_t;
    if (PEN && ((L.bitmap[(e0 - c0) >> 5] >> (((e0 - c0) & 31) + j)) & 1u)) v = -INFINITY;
    if (MASK && !((bt.mw[u] >> ((e0 & 31) + j)) & 1u)) v = -INFINITY;
    return is_invalid(v) ? -INFINITY : v;
  };

  // history ids first, so that the set-up waits for them and not for the logits
  int32_t hid[HIDR];
  if (PEN) {
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
#pragma unroll
    for (int r = 0; r < HIDR; ++r) {
      const int j = t + r * kBlock;
      const int32_t v = h[j < a.H ? j : a.H - 1];  // every lane loads: the loads in flight stay countable
      hid[r] = j < a.H ? v : -1;
    }
  }
  // two batches per wave are in flight while the workgroup sets up
  Batch ba, bb;
  int ia = wave, ib = wave + kWaves;
  load(ia, ba);
  load(ib, bb);

  if (t == 0) {
    s.next_batch = 2 * kWaves;
    s.flags = 0u;
  }
  for (int i = t; i < (int)(4 * sizeof(KeyHist) / 4); i += kBlock) reinterpret_cast<uint32_t*>(L.kh)[i] = 0u;
  if (PEN) {
    for (int i = t; i < a.bitmap_words; i += kBlock) L.bitmap[i] = 0u;
    if (own_hist || hist_inline)
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
        if (own_hist || hist_inline) hist_insert(L.htab, (uint32_t)a.hash_bits, (uint32_t)id);
      }
    }
    if (bad) atomicOr(&s.flags, kFlagBadHistory);
  }
  __syncthreads();

  bool bad = false;

  // ---- A. threshold T0: a lower bound of the k-th largest of the 1024 lane maxima of
  // the first two batches (the k-th largest of a subset never exceeds the k-th largest of
  // the whole): histogram of the order keys' top 10 bits, then of the next 10 bits in the
  // bin that holds the k-th; every wave reads the bins itself ----
  float t0;
  {
    float lm = -INFINITY;
#pragma unroll
    for (int q = 0; q < NQ; ++q) lm = fmaxf(lm, zsample(ia, ba, q));
#pragma unroll
    for (int q = 0; q < NQ; ++q) lm = fmaxf(lm, zsample(ib, bb, q));
    const uint32_t key = order_key(lm + 0.0f);
    key_hist_add(L.kh[0], key >> (32 - kBinBits));
    __syncthreads();
    uint32_t above1, above2;
    const int b1 = key_hist_kth(L.kh[0], (uint32_t)k, &above1);
    if ((int)(key >> (32 - kBinBits)) == b1) key_hist_add(L.kh[1], (key >> (32 - 2 * kBinBits)) & (kBins - 1));
    __syncthreads();
    const int b2 = key_hist_kth(L.kh[1], (uint32_t)k - above1, &above2);
    // lower edge of the bin: no key in it is smaller; -inf / NaN edges become -FLT_MAX
    t0 = fmaxf(key_value(((uint32_t)b1 << (32 - kBinBits)) | ((uint32_t)b2 << (32 - 2 * kBinBits))), -FLT_MAX);
  }

  // ---- B. stream: batches from an LDS counter, two in flight per wave ----
  uint64_t* buf = L.wb + wave * kTopkWaveCap;
  uint32_t* rh = L.hist + wave * 256;
  uint64_t* side = L.side + wave * kWave;
  int wc = 0, nside = 0;
  // append z >= thr. The raw test x >= x_thr is implied by z = fl(x * (1/T)) >= thr
  // (x_thr = thr * T lowered by a relative and an absolute margin), so the hot loop
  // compares raw logits and computes z only for the few that pass.
  float thr = 0.0f, x_thr = 0.0f;
  auto set_thr = [&](float t) {
    thr = uniform(t);
    const float tt = thr * a.temp;
    x_thr = uniform(tt - (fabsf(tt) * 0x1p-20f + 0x1p-120f));
  };
  set_thr(t0);
  bool ovf = false;
  auto grab = [&]() -> int {
    int b = 0;
    if (lane == 0) b = atomicAdd(&s.next_batch, 1);
    return lane_get(b, 0);
  };
  auto id_of = [&](int b, int q) { return c0 + (b * kBatch + (q / VEC) * kWave + lane) * VEC + (q % VEC); };
  // element q of a batch is past the chunk or masked (mw: its unit's mask word)
  auto dropped_w = [&](int b, int q, uint32_t mw) -> bool {
    const int unit = b * kBatch + (q / VEC) * kWave + lane;
    if (unit >= n_units) return true;
    return MASK && !((mw >> (((c0 + unit * VEC) & 31) + (q % VEC))) & 1u);
  };
  auto in_history = [&](int b, int q) -> bool {
    const int off = (b * kBatch + (q / VEC) * kWave + lane) * VEC;
    return PEN && ((L.bitmap[off >> 5] >> ((off & 31) + (q % VEC))) & 1u);
  };
  // one candidate (its lane passed the raw test): z, or -inf if not taken (history ids
  // scored at set-up are not taken here)
  auto candidate = [&](int b, int q, float x, uint32_t mw) -> float {
    if (dropped_w(b, q, mw)) return -INFINITY;
    const float v = x * a.inv_t;
    if (is_invalid(v)) {
      bad = true;  // +inf, or overflow to +inf
      return -INFINITY;
    }
    if (PEN && !hist_inline && in_history(b, q)) return -INFINITY;
    return v;
  };
  auto append = [&](uint64_t* dst, int& n, bool tk, float v, int id) {
    const uint64_t m = __ballot(tk);
    if (tk) dst[n + lanes_below(m)] = composite(v + 0.0f, id);
    n = uniform<int>(n + __popcll(m));
  };
  auto process = [&](int b, const Batch& bt) {
    uint64_t bal[NQ];
    uint64_t any = 0ull, nanm = 0ull;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const float x = unpack_unit<DT>(bt.w[q / VEC], q % VEC);
      if (MASK) {  // masked ids never pass (most ids of a constrained row are masked)
        const int e = c0 + (b * kBatch + (q / VEC) * kWave + lane) * VEC;
        bal[q] = __ballot(x >= x_thr && ((bt.mw[q / VEC] >> ((e & 31) + (q % VEC))) & 1u));
      } else {
        bal[q] = __ballot(x >= x_thr);
      }
      any |= bal[q];
      nanm |= __ballot(x != x);
    }
    if (nanm) {  // rare: a NaN counts unless masked or past the chunk
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const float x = unpack_unit<DT>(bt.w[q / VEC], q % VEC);
        if (x != x && !dropped_w(b, q, MASK ? bt.mw[q / VEC] : 0u)) bad = true;
      }
    }
    if (!any) return;
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < NQ; ++q) cnt += __popcll(bal[q]);
    if (wc + cnt <= kTopkWaveCap) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        if (!bal[q]) continue;
        bool tk = (bal[q] >> lane) & 1ull;
        float v = -INFINITY;
        if (tk) {
          v = candidate(b, q, unpack_unit<DT>(bt.w[q / VEC], q % VEC), MASK ? bt.mw[q / VEC] : 0u);
          tk = v >= thr;
        }
        const bool hist = hist_inline && tk && in_history(b, q);  // set aside, penalised at the end
        append(buf, wc, tk && !hist, v, id_of(b, q));
        if (PEN && __ballot(tk && hist)) {
          if (nside + __popcll(__ballot(tk && hist)) > kWave) {
            ovf = true;  // more than 64 history ids of one wave above the threshold: row solver
          } else {
            append(side, nside, tk && hist, v, id_of(b, q));
          }
        }
      }
      return;
    }
    // a batch that may not fit: one element slot at a time (picked by selects, so that
    // the buffer cut below exists once), the buffer cut to its k best when needed
#pragma unroll 1
    for (int q = 0; q < NQ; ++q) {
      float x = 0.0f;
      uint32_t mw = 0u;
      bool tk = false;
#pragma unroll
      for (int qq = 0; qq < NQ; ++qq) {
        if (qq == q) {
          x = unpack_unit<DT>(bt.w[qq / VEC], qq % VEC);
          mw = MASK ? bt.mw[qq / VEC] : 0u;
          tk = (bal[qq] >> lane) & 1ull;
        }
      }
      if (!__ballot(tk)) continue;
      float v = -INFINITY;
      if (tk) {
        v = candidate(b, q, x, mw);
        tk = v >= thr;
      }
      const bool hist = hist_inline && tk && in_history(b, q);
      if (wc + __popcll(__ballot(tk && !hist)) > kTopkWaveCap) {
        if (wc > k) set_thr(fmaxf(thr, wave_keep_topk<kTopkWaveCap>(buf, wc, k, rh)));
        tk = tk && v >= thr;
        if (wc + __popcll(__ballot(tk && !hist)) > kTopkWaveCap) {
          ovf = true;  // unreachable for k <= 64: the row would go to the row solver
          return;
        }
      }
      append(buf, wc, tk && !hist, v, id_of(b, q));
      if (PEN && __ballot(tk && hist)) {
        if (nside + __popcll(__ballot(tk && hist)) > kWave)
          ovf = true;
        else
          append(side, nside, tk && hist, v, id_of(b, q));
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
  // ---- C. history ids a penalty may raise (the row's first chunk scores all of them),
  // the history ids set aside while streaming, then the chunk's k best ----
  if (own_hist) {
    for (int r = 0; r * kBlock < (1 << a.hash_bits); ++r) {
      const int slot = t + r * kBlock;
      const uint32_t e = slot < (1 << a.hash_bits) ? L.htab[slot] : kEmptySlot;
      const int id = e != kEmptySlot ? (int)(e >> 12) : -1;
      float z = -INFINITY;
      if (id >= 0) {
        z = penalize(Elem<DT>::one(xrow, id) * a.inv_t + 0.0f, (e & 4095u) + 1u, a.pen);
        if (MASK && !((mrow[id >> 5] >> (id & 31)) & 1u)) z = -INFINITY;
        if (is_invalid(z)) {
          bad = true;
          z = -INFINITY;
        }
      }
      bool tk = z >= thr;
      if (wc + __popcll(__ballot(tk)) > kTopkWaveCap) {
        if (wc > k) set_thr(fmaxf(thr, wave_keep_topk<kTopkWaveCap>(buf, wc, k, rh)));
        tk = z >= thr;
      }
      append(buf, wc, tk, z, id);
    }
  }
  if (hist_inline && nside > 0) {  // history ids set aside: penalised now
    wave_lds_sync();
    const uint64_t c = lane < nside ? side[lane] : 0ull;
    float z = -INFINITY;
    const int id = composite_id(c);
    if (c != 0ull) z = penalize(composite_z(c), hist_count(L.htab, (uint32_t)a.hash_bits, (uint32_t)id), a.pen);
    bool tk = z >= thr;
    uint64_t bal = __ballot(tk);
    if (wc + __popcll(bal) > kTopkWaveCap) {
      if (wc > k) set_thr(fmaxf(thr, wave_keep_topk<kTopkWaveCap>(buf, wc, k, rh)));
      tk = z >= thr;
      bal = __ballot(tk);
    }
    if (tk) buf[wc + lanes_below(bal)] = composite(z, id);
    wc = uniform<int>(wc + __popcll(bal));
  }
  if (__ballot(bad) && lane == 0) atomicOr(&s.flags, kFlagInvalid);
  if (__ballot(ovf) && lane == 0) atomicOr(&s.flags, kFlagOverflow);

  // Final selection: the bin (20 bits of the order key, two levels) that holds the chunk's
  // k-th best; everything at or above its lower edge is gathered. When that is at most
  // 64 entries (no wide tie at the edge) one sort finishes the chunk; otherwise every
  // wave keeps its k best and a tree of bitonic merges combines the waves.
  if (t == 0) s.n_sel = 0;
  wave_lds_sync();
  constexpr int RB = kTopkWaveCap / kWave;
  uint64_t cv[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    cv[r] = r * kWave + lane < wc ? buf[r * kWave + lane] : 0ull;
    if (cv[r] != 0ull) key_hist_add(L.kh[2], (uint32_t)(cv[r] >> (64 - kBinBits)));
  }
  __syncthreads();
  const uint32_t total = wave_sum(L.kh[2].coarse[lane]);
  const uint32_t need = (uint32_t)k < total ? (uint32_t)k : total;
  uint64_t edge = 0ull;
  if (need > 0u) {
    uint32_t fa1, fa2;
    const int fb1 = key_hist_kth(L.kh[2], need, &fa1);
#pragma unroll
    for (int r = 0; r < RB; ++r)
      if (cv[r] != 0ull && (int)(cv[r] >> (64 - kBinBits)) == fb1)
        key_hist_add(L.kh[3], (uint32_t)(cv[r] >> (64 - 2 * kBinBits)) & (kBins - 1));
    __syncthreads();
    const int fb2 = key_hist_kth(L.kh[3], need - fa1, &fa2);
    edge = ((uint64_t)fb1 << (64 - kBinBits)) | ((uint64_t)fb2 << (64 - 2 * kBinBits));
  } else {
    __syncthreads();
  }
  {
    int ns = 0;
#pragma unroll
    for (int r = 0; r < RB; ++r) ns += __popcll(__ballot(cv[r] != 0ull && cv[r] >= edge));
    int base = 0;
    if (lane == 0 && ns > 0) base = atomicAdd(&s.n_sel, ns);
    base = lane_get(base, 0);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const bool in = cv[r] != 0ull && cv[r] >= edge;
      const uint64_t m = __ballot(in);
      const int pos = base + lanes_below(m);
      if (in && pos < kWave) L.sel[pos] = cv[r];
      base += __popcll(m);
    }
  }
  __syncthreads();
  uint32_t flags = s.flags;
  const int n_sel = s.n_sel;
  if (n_sel <= kWave && !((flags & kFlagOverflow) && !(flags & (kFlagBadHistory | kFlagInvalid)))) {
    if (wave != 0) return;
    uint64_t v = lane < n_sel ? L.sel[lane] : 0ull;
    v = wave_sort64_desc(v);
    const int n = min(k, n_sel);
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
    return;
  }

  if (wc > kWave) set_thr(fmaxf(thr, wave_keep_topk<kTopkWaveCap>(buf, wc, k, rh)));
  wave_lds_sync();
  uint64_t v = lane < wc ? buf[lane] : 0ull;
  v = wave_sort64_desc(v);

  // the list of wave w lives in the first 64 slots of its buffer
  uint64_t* lists = L.wb;
#pragma unroll
  for (int step = 1; step < kWaves; step <<= 1) {

    if ((wave & (2 * step - 1)) == step) lists[wave * kTopkWaveCap + lane] = v;
    __syncthreads();
    if (step == 1) {
      flags = s.flags;
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
    }
    if ((wave & (2 * step - 1)) == 0) v = list_merge(v, lists[(wave + step) * kTopkWaveCap + lane]);
  }
  if (wave != 0) return;
  const int n = min(k, list_count(v));
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
    pl.lds_stream = pl.mode_k ? arbor::TopkLds::bytes(pl.bitmap_words, p->hist_len > 0 ? (1 << hb) : 0)
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

// Raises a kernel's dynamic LDS limit to at least `lds` bytes. The attribute call costs
// microseconds of host time, so the limit set for each (kernel, device) is remembered and
// the call is made only when a launch needs more.
int allow_lds(const void* kernel, size_t lds) {
  static std::mutex mu;
  static const void* fns[512];
  static int devs[512];
  static size_t lims[512];
  static int n = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  int slot = -1;
  for (int i = 0; i < n; ++i)
    if (fns[i] == kernel && devs[i] == dev) slot = i;
  if (slot >= 0 && lims[slot] >= lds) return ARBOR_OK;
  hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute");
  if (slot < 0 && n < 512) slot = n++;
  if (slot >= 0) {
    fns[slot] = kernel;
    devs[slot] = dev;
    lims[slot] = lds;
  }
  return ARBOR_OK;
}

template <typename K>
int launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, const arbor::Args& a) {
  if (lds > 64 * 1024) {
    const int r = allow_lds(reinterpret_cast<const void*>(kernel), lds);
    if (r != ARBOR_OK) return r;
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
  a.temp = p->temperature;
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
  a.pen_mono = p->repetition_penalty >= 1.0f && p->frequency_penalty >= 0.0f && p->presence_penalty >= 0.0f;
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
