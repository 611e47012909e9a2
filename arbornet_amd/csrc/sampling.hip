// sampling.hip -- MI355X (gfx950) token-sampling kernels and the extern "C" ABI of
// libarbor_hip.so (declared in include/arbor_sampling.h).
//
// Two device paths compute the same contract:
//
//  * streaming top-k path (top-k <= 64, or min-p as the only filter, whose band the
//    64-entry list then holds): one 1024-thread workgroup per row (or, when the batch is
//    smaller than the chip, per chunk of a row) reads the row from HBM exactly once;
//    fifteen waves stream and queue candidates above a rising threshold, the sixteenth
//    keeps the best 64 and draws in fp64 (topk_stream.hpp, topk_path.hpp). Chunks of a
//    split row are merged by topk_finish_kernel.
//
//  * row solver (top-p without top-k, plain sampling, top-k > 64): mass_solver.hpp, with
//    the radix solver of row_solver.hpp as the fallback for heavily tied rows and for
//    streamed rows whose candidate list could not hold the answer.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <cmath>
#include <mutex>

#include "../../include/arbor_sampling.h"
#include "args.hpp"
#include "block_ops.hpp"
#include "lm_head.hpp"
#include "mass_solver.hpp"
#include "nucleus.hpp"
#include "row_solver.hpp"
#include "split_solver.hpp"
#include "tokens.hpp"
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

// Finishes top-k rows that were split into chunks: wave 0 of a workgroup per row merges
// the chunks' lists and draws; a row with an overflowed chunk is solved exactly.
template <int DT>
__global__ void __launch_bounds__(kBlock) topk_finish_kernel(Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SolverShared ssh;
  __shared__ uint32_t s_flags;
  const int lane = lane_id(), row = blockIdx.x;
  // wave 0 requests every chunk's count, flags and 64 list slots in one round (slots past
  // a chunk's count hold stale keys and are masked once the counts are in)
  constexpr int kGroup = 8;  // chunks merged per round of loads
  uint64_t v0[kGroup];
  uint32_t n0 = 0u;
  if (threadIdx.x < kWave) {
    uint32_t f = 0u;
    if (lane < a.S) {
      const size_t slot = (size_t)row * (size_t)a.S + (size_t)lane;
      n0 = a.hdr[slot * 2 + 0];
      f = a.hdr[slot * 2 + 1];
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j)
      v0[j] = j < a.S ? a.cand[((size_t)row * (size_t)a.S + (size_t)j) * kChunkSlot + lane] : 0ull;
    f = wave_reduce(f, [](uint32_t x, uint32_t y) { return x | y; });
    if (lane == 0) s_flags = f;
  }
  __syncthreads();
  const uint32_t flags = s_flags;
  // min-p band rows (top_k 0) go to the band solver, from the merged list's top (a chunk
  // that overflowed published nothing, so the solver checks that top against the row)
  __shared__ uint32_t s_top;
  const bool band = a.top_k == 0;
  uint32_t* htab = reinterpret_cast<uint32_t*>(smem);
  unsigned char* band_lds = smem + (sizeof(uint32_t) << a.hash_bits);
  const bool whole = a.aligned && a.V % Elem<DT>::kVec == 0;
  if ((flags & kFlagOverflow) && !(flags & (kFlagBadHistory | kFlagInvalid))) {
    if (band && whole)
      solve_band_row<kBlock, DT, true>(a, row, 0u, htab, band_lds);
    else if (band)
      solve_band_row<kBlock, DT, false>(a, row, 0u, htab, band_lds);
    else
      solve_row<kBlock, DT>(a, row, htab, ssh);
    return;
  }
  // wave 0 merges the chunks' lists; with min-p as the only filter (top_k 0) the merged
  // 64-entry list must hold the whole band, or the row is solved exactly
  __shared__ int s_exact;
  uint64_t best = 0ull;
  if (threadIdx.x < kWave) {
#pragma unroll
    for (int j = 0; j < kGroup; ++j)
      if (j < a.S) best = list_merge(best, lane < (int)lane_get(n0, j) ? v0[j] : 0ull);
    // more than kGroup chunks (rows of more than 8 chunks): the rest, kGroup at a time
    for (int cb = kGroup; cb < a.S; cb += kGroup) {
      uint64_t v[kGroup];
#pragma unroll
      for (int j = 0; j < kGroup; ++j) {
        const int c = cb + j;
        v[j] = 0ull;
        if (c < a.S) {
          const size_t slot = (size_t)row * (size_t)a.S + (size_t)c;
          const int n = (int)a.hdr[slot * 2 + 0];
          if (lane < n) v[j] = a.cand[slot * kChunkSlot + lane];
        }
      }
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
        if (cb + j < a.S) best = list_merge(best, v[j]);
    }
    const uint64_t last = lane_get(best, kWave - 1), top = lane_get(best, 0);
    if (lane == 0) {
      s_exact = band && last != 0ull && composite_z(last) >= composite_z(top) + a.ln_min_p_lo &&
                !(flags & (kFlagBadHistory | kFlagInvalid));
      s_top = (uint32_t)(top >> 32);
    }
  }
  __syncthreads();
  if (s_exact) {
    if (whole)
      solve_band_row<kBlock, DT, true>(a, row, s_top, htab, band_lds);
    else
      solve_band_row<kBlock, DT, false>(a, row, s_top, htab, band_lds);
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

// One generation step's history update, for the paths whose kernels do not append
// themselves: each row's sampled id (sentinels excluded) goes to slot positions[b] mod H of
// the row's ring, and positions[b] advances. Penalties count occurrences, so the ring's
// order does not matter.
__global__ void append_kernel(int32_t* history, int H, int32_t* positions, const int32_t* ids, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int32_t id = ids[b];
  if (id < 0) return;
  const uint32_t pos = (uint32_t)positions[b];
  history[(size_t)b * (size_t)H + pos % (uint32_t)H] = id;
  positions[b] = (int32_t)(pos + 1u);
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

enum class Path { Stream, Nucleus, Solver };

struct Plan {
  Path path;
  bool inline_fin;  // stream path: one chunk per row, finished in the same workgroup
  int k;            // effective top-k (0 = off)
  int S, chunk_len;
  int hash_bits, bitmap_words;
  size_t lds_stream, lds_solver, lds_nucleus;
  int mask_lds;  // byte offset of the LDS mask words (streamed masked rows), else -1
  size_t lds_finish;  // topk_finish_kernel: history table (+ the band solver's scratch)
  // workspace layout (byte offsets)
  size_t off_hdr, off_cand, off_zbuf, off_split, off_ctr, total;
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

// Compute units of the current device (256 on MI355X), cached per device. Concurrent
// first calls may both query the device; they store the same value atomically.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// The nucleus kernel's split: S workgroups per row when the batch is smaller than the chip,
// never below 16K ids per chunk; chunks of at most 262,144 ids (the history bitmap's reach).
void nucleus_geometry(const arbor_sampling_params* p, int cus, int hash_bits, int* S_out, int* len_out,
                      int* bitmap_words, size_t* lds) {
  const int V = p->vocab, B = p->batch;
  int S = B < cus ? cus / B : 1;
  const int by_len = (V + 16383) / 16384;
  if (S > by_len) S = by_len;
  if (S > arbor::kMaxChunks) S = arbor::kMaxChunks;
  const int by_bitmap = (V + arbor::kNuMaxChunk - 1) / arbor::kNuMaxChunk;
  if (S < by_bitmap) S = by_bitmap;
  if (S < 1) S = 1;
  const int len = (int)align_up((size_t)((V + S - 1) / S), 1024);
  *S_out = (V + len - 1) / len;
  *len_out = len;
  const int n_batches = (len + arbor::kNuBatchIds - 1) / arbor::kNuBatchIds;
  *bitmap_words = p->hist_len > 0 ? len / 32 : 0;
  *lds = (size_t)arbor::NuLayout::make(n_batches, *bitmap_words, p->hist_len > 0 ? (1 << hash_bits) : 0).bytes;
}

Plan make_plan(const arbor_sampling_params* p, int cus) {
  Plan pl{};
  const int V = p->vocab, B = p->batch;
  pl.k = (p->top_k > 0 && p->top_k < V) ? p->top_k : 0;
  // the streaming top-k kernel: top-k <= 64, or min-p as the only filter (its 64-entry
  // list then holds the min-p band); without top-k otherwise (top-p, with or without min-p,
  // or no filter at all) the two-pass nucleus kernel; top-k above 64 the histogram solver
  const bool minp_only = pl.k == 0 && p->top_p >= 1.0f && p->min_p > 0.0f;
  pl.path = (pl.k > 0 && pl.k <= arbor::kMaxTopK) || minp_only ? Path::Stream
            : pl.k == 0                                           ? Path::Nucleus
                                                                  : Path::Solver;
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
    pl.lds_stream = arbor::TkLds::bytes(pl.bitmap_words, p->hist_len > 0 ? (1 << hb) : 0);
  } else if (pl.path == Path::Nucleus) {
    nucleus_geometry(p, cus, hb, &pl.S, &pl.chunk_len, &pl.bitmap_words, &pl.lds_nucleus);
  } else if (B < cus) {
    // row solver over S workgroups per row, never below 8K ids per chunk
    int S = cus / B;
    const int by_len = (V + 8191) / 8192;
    if (S > by_len) S = by_len;
    if (S > 1) {
      const int len = (int)align_up((size_t)((V + S - 1) / S), 512);
      pl.S = (V + len - 1) / len;
      pl.chunk_len = len;
    }
  }
  pl.lds_solver = sizeof(uint32_t) * (size_t)(1 << hb);
  pl.lds_finish = pl.lds_solver + (pl.path == Path::Stream && pl.k == 0 ? arbor::band_lds_bytes(V, arbor::kBlock) : 0);
  size_t off = 0;
  // Workspace per path: split streamed rows publish each chunk's list (count, flags and 64
  // candidates); the histogram solvers keep one padded fp32 z row per row (and, split, one
  // record per workgroup and the barrier counters). Rows streamed whole need nothing: their
  // exact fallback recomputes z from the logits.
  const bool chunk_lists = pl.path == Path::Stream && pl.S > 1;
  pl.off_hdr = off;
  if (chunk_lists) off = align_up(off + sizeof(uint32_t) * 2 * (size_t)B * (size_t)pl.S, 256);
  pl.off_cand = off;
  if (chunk_lists) off = align_up(off + sizeof(uint64_t) * arbor::kChunkSlot * (size_t)B * (size_t)pl.S, 256);
  pl.off_zbuf = off;
  if (pl.path == Path::Solver) off = align_up(off + sizeof(float) * (size_t)B * align_up((size_t)V, 64), 256);
  pl.off_split = off;
  pl.off_ctr = off;
  if (pl.path == Path::Solver && pl.S > 1) {
    off = align_up(off + sizeof(arbor::SplitChunk) * (size_t)B * (size_t)pl.S, 256);
    pl.off_ctr = off;
    off = align_up(off + sizeof(uint32_t) * (2 * (size_t)B + 1), 256);  // row barriers, ticket, failure words
  }
  if (pl.path == Path::Nucleus && pl.S > 1) {
    off = align_up(off + sizeof(arbor::NuRec) * (size_t)B * (size_t)pl.S, 256);
    pl.off_ctr = off;
    off = align_up(off + sizeof(uint64_t) * (2 * (size_t)B), 256);  // tagged barrier and failure words
  }
  pl.total = off > 256 ? off : 256;  // never 0: 0 reports invalid params
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

template <int DT, bool PEN, bool MASK, bool ALIGNED, bool BAND>
int launch_topk5(const Plan& pl, hipStream_t st, const arbor::Args& a) {
  const dim3 grid((unsigned)(a.B * pl.S)), block(arbor::kTkBlock);
  if constexpr (ALIGNED && !MASK) {
    // rows the plan finishes in one workgroup and that fit one round of requests
    if (pl.S == 1 && a.V <= arbor::tk_whole_max_ids(arbor::Elem<DT>::kVec))
      return launch(arbor::topk_kernel<DT, PEN, false, true, true, BAND, true>, grid, block, pl.lds_stream, st, a);
  }
  int r = pl.inline_fin
              ? launch(arbor::topk_kernel<DT, PEN, MASK, true, ALIGNED, BAND>, grid, block, pl.lds_stream, st, a)
              : launch(arbor::topk_kernel<DT, PEN, MASK, false, ALIGNED, BAND>, grid, block, pl.lds_stream, st, a);
  if (r != ARBOR_OK || pl.inline_fin) return r;
  return launch(arbor::topk_finish_kernel<DT>, dim3((unsigned)a.B), dim3(arbor::kBlock), pl.lds_finish, st, a);
}

// min-p as the only filter (top_k 0) compiles the band rules in
template <int DT, bool PEN, bool MASK, bool ALIGNED>
int launch_topk4(const Plan& pl, hipStream_t st, const arbor::Args& a) {
  if (pl.k == 0) return launch_topk5<DT, PEN, MASK, ALIGNED, true>(pl, st, a);
  return launch_topk5<DT, PEN, MASK, ALIGNED, false>(pl, st, a);
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

// Whether the split row solver's grid can be resident at once on the current device
// (enough workgroup slots, so that every row's workgroups run together on an idle device;
// the kernel's ticket order keeps it correct with fewer); cached per device and size.
bool split_fits(const void* kernel, size_t lds, int blocks) {
  static std::mutex mu;
  static const void* fns[64];
  static int devs[64], nblk[64];
  static size_t ldss[64];
  static int n = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n; ++i)
    if (fns[i] == kernel && devs[i] == dev && ldss[i] == lds) return nblk[i] >= blocks;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, arbor::kBlock, lds) != hipSuccess) per_cu = 0;
  const int total = per_cu * device_cus();
  if (n < 64) {
    fns[n] = kernel;
    devs[n] = dev;
    ldss[n] = lds;
    nblk[n] = total;
    ++n;
  }
  return total >= blocks;
}

// Spin limit of the split solver's row barriers: kSplitSpinLimit (seconds of waiting), or
// ARBOR_SPLIT_SPIN_LIMIT from the environment. Tests set a tiny limit to exercise the
// give-up path (every kernel still ends: a wait that gives up stops waiting).
uint32_t split_spin_limit() {
  const char* env = getenv("ARBOR_SPLIT_SPIN_LIMIT");
  if (env && *env) {
    const unsigned long v = strtoul(env, nullptr, 10);
    if (v > 0 && v < arbor::kSplitSpinLimit) return (uint32_t)v;
  }
  return arbor::kSplitSpinLimit;
}

// The two-pass nucleus kernel: one instance per (dtype, whole aligned units, history, mask).
// Split rows meet at barriers whose words carry a per-call tag, taken from a counter shared
// by every call of the process, so the workspace needs no clearing between calls.
uint32_t next_call_tag() {
  static std::atomic<uint32_t> tag{0};
  uint32_t t = tag.fetch_add(1u, std::memory_order_relaxed) + 1u;
  if (t == 0u) t = tag.fetch_add(1u, std::memory_order_relaxed) + 1u;  // 0 never tags a call
  return t;
}

template <int DT, bool ALIGNED, bool PEN, bool MASK>
int launch_nucleus4(const Plan& pl, hipStream_t st, const arbor::Args& a, char* ws) {
  auto kernel = arbor::nucleus_kernel<DT, ALIGNED, PEN, MASK>;
  if (pl.lds_nucleus > 64 * 1024) {
    const int r = allow_lds(reinterpret_cast<const void*>(kernel), pl.lds_nucleus);
    if (r != ARBOR_OK) return r;
  }
  arbor::NuRec* recs = pl.S > 1 ? reinterpret_cast<arbor::NuRec*>(ws + pl.off_split) : nullptr;
  uint64_t* ctr = pl.S > 1 ? reinterpret_cast<uint64_t*>(ws + pl.off_ctr) : nullptr;
  hipLaunchKernelGGL(kernel, dim3((unsigned)(a.B * pl.S)), dim3(arbor::kNuBlock), pl.lds_nucleus, st, a, recs, ctr,
                     next_call_tag(), split_spin_limit());
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return ARBOR_OK;
}

template <int DT, bool ALIGNED>
int launch_nucleus2(const Plan& pl, bool pen, bool mask, hipStream_t st, const arbor::Args& a, char* ws) {
  if (pen) return mask ? launch_nucleus4<DT, ALIGNED, true, true>(pl, st, a, ws)
                       : launch_nucleus4<DT, ALIGNED, true, false>(pl, st, a, ws);
  return mask ? launch_nucleus4<DT, ALIGNED, false, true>(pl, st, a, ws)
              : launch_nucleus4<DT, ALIGNED, false, false>(pl, st, a, ws);
}

template <int DT>
int launch_nucleus(const Plan& pl, bool pen, bool mask, hipStream_t st, const arbor::Args& a, char* ws) {
  // whole 16-byte units only: aligned rows whose length is a multiple of the unit
  if (a.aligned && a.V % arbor::Elem<DT>::kVec == 0) return launch_nucleus2<DT, true>(pl, pen, mask, st, a, ws);
  return launch_nucleus2<DT, false>(pl, pen, mask, st, a, ws);
}

// The row solver: S workgroups per row when the plan splits rows and the grid can be
// resident at once, else one workgroup per row.
template <int DT>
int launch_solver(const Plan& pl, hipStream_t st, arbor::Args a, char* ws) {
  const size_t lds = arbor::solver_lds_bytes(pl.hash_bits);
  const void* split = reinterpret_cast<const void*>(arbor::split_solver_kernel<DT>);
  if (pl.S > 1) {
    if (lds > 64 * 1024) {
      const int r = allow_lds(split, lds);
      if (r != ARBOR_OK) return r;
    }
    if (split_fits(split, lds, a.B * pl.S)) {
      arbor::SplitChunk* chunks = reinterpret_cast<arbor::SplitChunk*>(ws + pl.off_split);
      uint32_t* ctr = reinterpret_cast<uint32_t*>(ws + pl.off_ctr);
      // the rows' barrier counters, the ticket counter and the rows' failure words start at
      // zero (a fill kernel: no memset node in a captured graph)
      const int nctr = 2 * a.B + 1;
      hipLaunchKernelGGL(arbor::zero_u32_kernel, dim3((unsigned)((nctr + 255) / 256)), dim3(256), 0, st, ctr, nctr);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return hip_fail(e, "kernel launch");
      hipLaunchKernelGGL(arbor::split_solver_kernel<DT>, dim3((unsigned)(a.B * pl.S)), dim3(arbor::kBlock), lds, st, a,
                         chunks, ctr, split_spin_limit());
      e = hipGetLastError();
      if (e != hipSuccess) return hip_fail(e, "kernel launch");
      return ARBOR_OK;
    }
  }
  return launch(arbor::solver_kernel<DT>, dim3((unsigned)a.B), dim3(arbor::kBlock), lds, st, a);
}

// ---------------------------------------------------------------------------------------
// Static scratch of arbor_sample_noalloc: the workspace of callers that cannot allocate.
// Every device the library runs on holds its own copy until the process ends. In host code
// `scratch` names a host-side stand-in, not device memory: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only that address
// is ever handed to a kernel.
// ---------------------------------------------------------------------------------------
constexpr size_t kScratchBytes = ARBOR_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(ARBOR_ERR_NO_DEVICE, "device %d beyond the %d this library serves", dev,
                                                 kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(ARBOR_ERR_NO_DEVICE, "hipGetSymbolAddress(scratch) returned NULL");
    addr[dev] = p;
  }
  *out = addr[dev];
  return ARBOR_OK;
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

// Appends every row's sampled id to its history ring, for kernels that do not append
// themselves.
static int launch_append(const arbor_sampling_params* p, hipStream_t s, int32_t* ring_hist, int32_t* ring_pos,
                         const int32_t* out_ids) {
  hipLaunchKernelGGL(arbor::append_kernel, dim3((unsigned)((p->batch + 255) / 256)), dim3(256), 0, s, ring_hist,
                     (int)p->hist_len, ring_pos, out_ids, (int)p->batch);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return ARBOR_OK;
}

// arbor_sample's body; with ring_pos set (a generation step) it also appends each row's id
// to the row's history ring. Kernels that finish a row in one workgroup append it
// themselves, after the row's history was read; rows finished by split workgroups (which
// may still end ARBOR_ID_STALLED after another chunk drew) are appended by a second launch.
static int sample_impl(const arbor_sampling_params* p, const void* logits, const int32_t* history,
                       const uint32_t* allow_mask, const float* uniforms, int32_t* out_ids, float* out_probs,
                       void* workspace, size_t workspace_bytes, void* stream, int32_t* ring_hist, int32_t* ring_pos) {
  int st = validate(p);
  if (st != ARBOR_OK) return st;
  if (!logits || !uniforms || !out_ids) return fail(ARBOR_ERR_NULL, "logits, uniforms and out_ids are required");
  if (p->hist_len > 0 && !history) return fail(ARBOR_ERR_HISTORY, "history is NULL with hist_len %d", p->hist_len);
  if (allow_mask && p->mask_words < (p->vocab + 31) / 32)
    return fail(ARBOR_ERR_MASK, "mask_words %d < ceil(vocab / 32) = %d", p->mask_words, (p->vocab + 31) / 32);
  const bool probs = (p->flags & ARBOR_FLAG_WRITE_PROBS) != 0;
  if (probs && !out_probs) return fail(ARBOR_ERR_FLAGS, "ARBOR_FLAG_WRITE_PROBS without out_probs");
  Plan pl = make_plan(p, device_cus());
  // masked streamed fp32 rows keep the chunk's allow-mask words in LDS (after the history
  // table), so a unit's mask is known before its logits are requested
  pl.mask_lds = -1;
  if (allow_mask && pl.path == Path::Stream && p->dtype == ARBOR_DTYPE_F32) {
    pl.mask_lds = (int)pl.lds_stream;
    // the mask words, then the list of the units that hold an allowed id
    pl.lds_stream += sizeof(uint32_t) * (size_t)(pl.chunk_len / 32) + sizeof(uint16_t) * arbor::kTkUnitList;
  }
  if (!workspace || workspace_bytes < pl.total)
    return fail(ARBOR_ERR_WORKSPACE, "workspace of %zu bytes given, %zu needed", workspace ? workspace_bytes : 0,
                pl.total);
  // short unmasked rows of whole aligned 16-byte units: one workgroup per row requests the
  // whole row at once (topk_kernel's WHOLE instances; the workspace the plan asked for
  // covers this, which needs none)
  {
    const size_t esz_ = p->dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
    const int vec = p->dtype == ARBOR_DTYPE_BF16 ? 8 : 4;
    const bool aligned_ = ((uintptr_t)logits % 16 == 0) && (((size_t)p->ld_logits * esz_) % 16 == 0);
    if (pl.path == Path::Stream && !allow_mask && aligned_ && p->vocab % vec == 0 &&
        p->vocab <= arbor::tk_whole_max_ids(vec)) {
      pl.S = 1;
      pl.chunk_len = (int)align_up((size_t)p->vocab, 512);
      pl.inline_fin = true;
      pl.bitmap_words = p->hist_len > 0 ? pl.chunk_len / 32 : 0;
      pl.lds_stream = arbor::TkLds::bytes(pl.bitmap_words, p->hist_len > 0 ? (1 << pl.hash_bits) : 0);
    }
  }

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
  a.ln_min_p = p->min_p > 0.0f ? log((double)p->min_p) : -INFINITY;
  a.S = pl.S;
  a.chunk_len = pl.chunk_len;
  a.hash_bits = pl.hash_bits;
  a.bitmap_words = pl.bitmap_words;
  a.mask_lds = pl.mask_lds;
  const size_t esz = p->dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
  a.aligned = ((uintptr_t)logits % 16 == 0) && (((size_t)p->ld_logits * esz) % 16 == 0);
  a.write_probs = probs ? 1 : 0;
  a.pen_mono = p->repetition_penalty >= 1.0f && p->frequency_penalty >= 0.0f && p->presence_penalty >= 0.0f;
  char* ws = static_cast<char*>(workspace);
  a.hdr = reinterpret_cast<uint32_t*>(ws + pl.off_hdr);
  a.cand = reinterpret_cast<uint64_t*>(ws + pl.off_cand);
  a.zbuf = reinterpret_cast<float*>(ws + pl.off_zbuf);
  a.ldz = (int)align_up((size_t)p->vocab, 64);
  const bool bf16 = p->dtype == ARBOR_DTYPE_BF16;
  const bool pen = p->hist_len > 0, mask = allow_mask != nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (pl.path == Path::Solver) {
    st = bf16 ? launch_solver<ARBOR_DTYPE_BF16>(pl, s, a, ws) : launch_solver<ARBOR_DTYPE_F32>(pl, s, a, ws);
    if (st != ARBOR_OK || !ring_pos) return st;
    return launch_append(p, s, ring_hist, ring_pos, out_ids);
  }
  if (pl.path == Path::Nucleus) {
    if (ring_pos && pl.S == 1) {
      a.ring_hist = ring_hist;
      a.ring_pos = ring_pos;
    }
    st = bf16 ? launch_nucleus<ARBOR_DTYPE_BF16>(pl, pen, mask, s, a, ws)
              : launch_nucleus<ARBOR_DTYPE_F32>(pl, pen, mask, s, a, ws);
    if (st != ARBOR_OK || !ring_pos || pl.S == 1) return st;
    return launch_append(p, s, ring_hist, ring_pos, out_ids);
  }
  // streamed rows: every row is finished by one workgroup (the streaming kernel's, or the
  // finishing kernel's for split rows), which appends it
  if (ring_pos) {
    a.ring_hist = ring_hist;
    a.ring_pos = ring_pos;
  }
  return bf16 ? launch_topk<ARBOR_DTYPE_BF16>(pl, pen, mask, s, a) : launch_topk<ARBOR_DTYPE_F32>(pl, pen, mask, s, a);
}

int arbor_sample(const arbor_sampling_params* p, const void* logits, const int32_t* history,
                 const uint32_t* allow_mask, const float* uniforms, int32_t* out_ids, float* out_probs,
                 void* workspace, size_t workspace_bytes, void* stream) {
  return sample_impl(p, logits, history, allow_mask, uniforms, out_ids, out_probs, workspace, workspace_bytes, stream,
                     nullptr, nullptr);
}

int arbor_sample_append(const arbor_sampling_params* p, const void* logits, int32_t* history, int32_t* positions,
                        const uint32_t* allow_mask, const float* uniforms, int32_t* out_ids, float* out_probs,
                        void* workspace, size_t workspace_bytes, void* stream) {
  int st = validate(p);
  if (st != ARBOR_OK) return st;
  if (p->hist_len <= 0 || !history || !positions)
    return fail(ARBOR_ERR_HISTORY, "a history ring (hist_len > 0) and positions are required");
  return sample_impl(p, logits, history, allow_mask, uniforms, out_ids, out_probs, workspace, workspace_bytes, stream,
                     history, positions);
}

int arbor_sample_noalloc(const arbor_sampling_params* p, const void* logits, const int32_t* history,
                         const uint32_t* allow_mask, const float* uniforms, int32_t* out_ids, float* out_probs,
                         void* stream) {
  int st = validate(p);
  if (st != ARBOR_OK) return st;
  const size_t need = make_plan(p, device_cus()).total;
  if (need > kScratchBytes)
    return fail(ARBOR_ERR_WORKSPACE,
                "these params need %zu bytes of workspace; the static scratch of arbor_sample_noalloc holds %zu "
                "(call arbor_sample with a workspace of arbor_sample_workspace_bytes() instead)",
                need, kScratchBytes);
  void* ws = nullptr;
  st = scratch_address(&ws);
  if (st != ARBOR_OK) return st;
  return arbor_sample(p, logits, history, allow_mask, uniforms, out_ids, out_probs, ws, kScratchBytes, stream);
}

int arbor_decode(const int32_t* ids, int32_t count, const int32_t* token_offsets, const uint8_t* token_bytes,
                 int32_t vocab, int32_t unk_id, int32_t* out_offsets, uint8_t* out_bytes, size_t out_capacity,
                 void* stream) {
  if (count < 0 || vocab < 0) return fail(ARBOR_ERR_SHAPE, "count %d and vocab %d must be >= 0", count, vocab);
  if (!out_offsets || (count > 0 && !ids) || (vocab > 0 && (!token_offsets || !token_bytes)) ||
      (out_capacity > 0 && !out_bytes))
    return fail(ARBOR_ERR_NULL, "ids, token_offsets, token_bytes, out_offsets and out_bytes are required");
  hipLaunchKernelGGL(arbor::decode_kernel, dim3(1), dim3(arbor::kDecodeBlock), 0, static_cast<hipStream_t>(stream),
                     ids, (int)count, token_offsets, token_bytes, (int)vocab, (int)unk_id, out_offsets, out_bytes,
                     out_capacity);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "kernel launch");
}

int arbor_embed(const int32_t* ids, int32_t count, const void* table, int32_t vocab, int32_t width, int32_t dtype,
                void* out_rows, void* stream) {
  if (count < 0 || vocab <= 0 || width <= 0)
    return fail(ARBOR_ERR_SHAPE, "count %d >= 0, vocab %d > 0 and width %d > 0 are required", count, vocab, width);
  if (dtype != ARBOR_DTYPE_F32 && dtype != ARBOR_DTYPE_BF16) return fail(ARBOR_ERR_DTYPE, "unknown dtype %d", dtype);
  if (count == 0) return ARBOR_OK;
  if (!ids || !table || !out_rows) return fail(ARBOR_ERR_NULL, "ids, table and out_rows are required");
  const size_t row_bytes = (size_t)width * (dtype == ARBOR_DTYPE_BF16 ? 2 : 4);
  if (row_bytes > (size_t)INT32_MAX) return fail(ARBOR_ERR_SHAPE, "rows of %zu bytes are too long", row_bytes);
  const bool units = row_bytes % 16 == 0 && (uintptr_t)table % 16 == 0 && (uintptr_t)out_rows % 16 == 0;
  const unsigned nx = (unsigned)((row_bytes / (units ? 16 : 1) + 255) / 256);
  const dim3 grid(units ? nx : (nx < 64u ? nx : 64u), (unsigned)count);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned char* tb = static_cast<const unsigned char*>(table);
  unsigned char* ob = static_cast<unsigned char*>(out_rows);
  if (units)
    hipLaunchKernelGGL(arbor::embed_kernel<true>, grid, dim3(256), 0, s, ids, tb, (int)vocab, (int)row_bytes, ob);
  else
    hipLaunchKernelGGL(arbor::embed_kernel<false>, grid, dim3(256), 0, s, ids, tb, (int)vocab, (int)row_bytes, ob);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "kernel launch");
}

size_t arbor_lm_head_packed_bytes(int32_t hidden, int32_t vocab) {
  if (hidden <= 0 || hidden % arbor::kLmHidden != 0 || vocab <= 0 || vocab > ARBOR_VOCAB_MAX) return 0;
  return arbor::lm_packed_bytes(hidden, vocab);
}

int arbor_lm_head_pack(const void* weight, int32_t weight_dtype, int32_t layout, int32_t hidden, int32_t vocab,
                       void* packed, void* stream) {
  if (arbor_lm_head_packed_bytes(hidden, vocab) == 0)
    return fail(ARBOR_ERR_SHAPE, "hidden %d must be a positive multiple of %d and vocab %d in (0, %d]", hidden,
                arbor::kLmHidden, vocab, ARBOR_VOCAB_MAX);
  if (weight_dtype != ARBOR_DTYPE_F32 && weight_dtype != ARBOR_DTYPE_BF16)
    return fail(ARBOR_ERR_DTYPE, "unknown weight dtype %d", weight_dtype);
  if (layout != ARBOR_LM_WEIGHT_HV && layout != ARBOR_LM_WEIGHT_VH)
    return fail(ARBOR_ERR_FLAGS, "unknown weight layout %d", layout);
  if (!weight || !packed) return fail(ARBOR_ERR_NULL, "weight and packed are required");
  if ((uintptr_t)packed % 16 != 0) return fail(ARBOR_ERR_SHAPE, "packed must be 16-byte aligned");
  const int rows = (int)((vocab + arbor::kLmRows - 1) / arbor::kLmRows * arbor::kLmRows);
  const size_t units = (size_t)rows * (size_t)(hidden / 8);
  const dim3 grid((unsigned)((units + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  arbor::lm_u4* out = static_cast<arbor::lm_u4*>(packed);
  if (weight_dtype == ARBOR_DTYPE_F32)
    hipLaunchKernelGGL(arbor::lm_pack_kernel<ARBOR_DTYPE_F32>, grid, dim3(256), 0, s, weight, (int)layout, (int)hidden,
                       (int)vocab, rows, out);
  else
    hipLaunchKernelGGL(arbor::lm_pack_kernel<ARBOR_DTYPE_BF16>, grid, dim3(256), 0, s, weight, (int)layout, (int)hidden,
                       (int)vocab, rows, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ARBOR_OK : hip_fail(e, "kernel launch");
}

}  // extern "C"

namespace {
template <int NT, int XDT>
void launch_lm_nt(const arbor::LmArgs& a, int odt, hipStream_t s) {
  const dim3 grid((unsigned)((a.V + arbor::kLmRows - 1) / arbor::kLmRows)), block(arbor::kLmThreads);
  if (odt == ARBOR_DTYPE_F32)
    hipLaunchKernelGGL((arbor::lm_head_kernel<NT, XDT, ARBOR_DTYPE_F32>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((arbor::lm_head_kernel<NT, XDT, ARBOR_DTYPE_BF16>), grid, block, 0, s, a);
}
template <int XDT>
void launch_lm(const arbor::LmArgs& a, int odt, hipStream_t s) {
  // batch rows in N-tiles of 32: 1, 2, 4 or 8 tiles
  const int nt = (a.B + 31) / 32;
  if (nt <= 1) launch_lm_nt<1, XDT>(a, odt, s);
  else if (nt <= 2) launch_lm_nt<2, XDT>(a, odt, s);
  else if (nt <= 4) launch_lm_nt<4, XDT>(a, odt, s);
  else launch_lm_nt<8, XDT>(a, odt, s);
}
}  // namespace

extern "C" {

int arbor_lm_head(const void* x, int32_t x_dtype, int32_t batch, int32_t ld_x, const void* packed, const float* bias,
                  int32_t hidden, int32_t vocab, float scale, void* logits, int32_t logits_dtype, int32_t ld_logits,
                  float* row_max, void* stream) {
  if (arbor_lm_head_packed_bytes(hidden, vocab) == 0)
    return fail(ARBOR_ERR_SHAPE, "hidden %d must be a positive multiple of %d and vocab %d in (0, %d]", hidden,
                arbor::kLmHidden, vocab, ARBOR_VOCAB_MAX);
  if (batch < 0 || ld_x < hidden || ld_logits < vocab)
    return fail(ARBOR_ERR_SHAPE, "batch %d >= 0, ld_x %d >= hidden %d and ld_logits %d >= vocab %d are required", batch,
                ld_x, hidden, ld_logits, vocab);
  if ((x_dtype != ARBOR_DTYPE_F32 && x_dtype != ARBOR_DTYPE_BF16) ||
      (logits_dtype != ARBOR_DTYPE_F32 && logits_dtype != ARBOR_DTYPE_BF16))
    return fail(ARBOR_ERR_DTYPE, "unknown dtype: x %d, logits %d", x_dtype, logits_dtype);
  if (!std::isfinite(scale)) return fail(ARBOR_ERR_TEMPERATURE, "scale must be finite, got %g", (double)scale);
  if (batch == 0) return ARBOR_OK;
  if (!x || !packed || !logits) return fail(ARBOR_ERR_NULL, "x, packed and logits are required");
  const size_t xe = x_dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
  if ((uintptr_t)x % 16 != 0 || ((size_t)ld_x * xe) % 16 != 0 || (uintptr_t)packed % 16 != 0)
    return fail(ARBOR_ERR_SHAPE, "x rows (ld_x %d) and packed must be 16-byte aligned", ld_x);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (row_max) {
    hipLaunchKernelGGL(arbor::lm_fill_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s, row_max,
                       (int)batch, -INFINITY);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
  }
  const size_t oe = logits_dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
  for (int b0 = 0; b0 < batch; b0 += arbor::kLmMaxB) {
    arbor::LmArgs a{};
    a.x = static_cast<const char*>(x) + (size_t)b0 * (size_t)ld_x * xe;
    a.ld_x = ld_x;
    a.w = static_cast<const arbor::lm_u4*>(packed);
    a.bias = bias;
    a.out = static_cast<char*>(logits) + (size_t)b0 * (size_t)ld_logits * oe;
    a.ld_out = ld_logits;
    a.row_max = row_max ? row_max + b0 : nullptr;
    a.scale = scale;
    a.B = batch - b0 < arbor::kLmMaxB ? batch - b0 : arbor::kLmMaxB;
    a.H = hidden;
    a.V = vocab;
    if (x_dtype == ARBOR_DTYPE_BF16)
      launch_lm<ARBOR_DTYPE_BF16>(a, logits_dtype, s);
    else
      launch_lm<ARBOR_DTYPE_F32>(a, logits_dtype, s);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
  }
  return ARBOR_OK;
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
