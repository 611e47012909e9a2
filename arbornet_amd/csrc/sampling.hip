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
#include "mass_solver.hpp"
#include "row_solver.hpp"
#include "topk_path.hpp"
#include "topk_stream.hpp"

namespace arbor {

// Dynamic LDS of solver_kernel: history table | FastShared.
__host__ __device__ constexpr size_t solver_lds_bytes(int hash_bits) {
  return ((sizeof(uint32_t) << hash_bits) + 15) / 16 * 16 + sizeof(FastShared);
}

template <int DT>
__global__ void __launch_bounds__(kBlock) solver_kernel(Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  FastShared& sh = *reinterpret_cast<FastShared*>(smem + ((sizeof(uint32_t) << a.hash_bits) + 15) / 16 * 16);
  solve_row_fast<kBlock, DT>(a, blockIdx.x, reinterpret_cast<uint32_t*>(smem), sh);
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
  // wave 0 merges the chunks' lists; with min-p as the only filter (top_k 0) the merged
  // 64-entry list must hold the whole band, or the row is solved exactly
  __shared__ int s_exact;
  uint64_t best = 0ull;
  if (threadIdx.x < kWave) {
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
    const uint64_t last = lane_get(best, kWave - 1), top = lane_get(best, 0);
    if (lane == 0)
      s_exact = a.top_k == 0 && last != 0ull && composite_z(last) >= composite_z(top) + a.ln_min_p_lo &&
                !(flags & (kFlagBadHistory | kFlagInvalid));
  }
  __syncthreads();
  if (s_exact) {
    solve_row<kBlock, DT>(a, row, reinterpret_cast<uint32_t*>(smem), ssh);
    return;
  }
  if (threadIdx.x >= kWave) return;
  const int n = min(a.top_k > 0 ? a.top_k : kWave, list_count(best));
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
  } else if (minp_only) {  // the top-k kernel's 64-entry list holds the min-p band
    pl.path = Path::Stream;
    pl.mode_k = true;
  } else {
    pl.path = Path::Solver;
  }
  int hb = 6;
  while ((1 << hb) < 2 * p->hist_len) ++hb;
  pl.hash_bits = hb;
  pl.S = 1;
  if (pl.path == Path::Stream) {
    // one workgroup per compute unit: split rows only when the batch is smaller than the
    // chip, and never below 8K ids per chunk
    int S = B < cus ? cus / B : 1;
    const int by_len = (V + 8191) / 8192;
    if (S > by_len) S = by_len;
    if (!pl.mode_k) {  // the min-p finish gathers every chunk's list in LDS
      const int slots = arbor::kWaves * arbor::kWaveCap / 2 / arbor::kChunkSlot;
      if (S > slots) S = slots;
    }
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
    pl.lds_stream = pl.mode_k ? arbor::TkLds::bytes(pl.bitmap_words, p->hist_len > 0 ? (1 << hb) : 0)
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
  off = align_up(off + sizeof(float) * (size_t)B * align_up((size_t)V, 64), 256);
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
  const dim3 grid((unsigned)(a.B * pl.S)), block(arbor::kTkBlock);
  int r = pl.inline_fin
              ? launch(arbor::topk_kernel<DT, PEN, MASK, true, ALIGNED>, grid, block, pl.lds_stream, st, a)
              : launch(arbor::topk_kernel<DT, PEN, MASK, false, ALIGNED>, grid, block, pl.lds_stream, st, a);
  if (r != ARBOR_OK || pl.inline_fin) return r;
  return launch(arbor::topk_finish_kernel<DT>, dim3((unsigned)a.B), dim3(arbor::kBlock), pl.lds_solver, st, a);
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
  a.ldz = (int)align_up((size_t)p->vocab, 64);
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (pl.path == Path::Solver) {
    const dim3 grid(p->batch), block(arbor::kBlock);
    const size_t lds = arbor::solver_lds_bytes(pl.hash_bits);
    if (p->dtype == ARBOR_DTYPE_BF16) return launch(arbor::solver_kernel<ARBOR_DTYPE_BF16>, grid, block, lds, s, a);
    return launch(arbor::solver_kernel<ARBOR_DTYPE_F32>, grid, block, lds, s, a);
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
