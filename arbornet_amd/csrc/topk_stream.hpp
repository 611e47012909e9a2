// topk_stream.hpp -- streaming top-k kernel (1 <= k <= 64): one 1024-thread workgroup per
// row, or per chunk of a row when the batch is smaller than the chip.
//
// Fifteen waves stream the row; the sixteenth, the finisher, keeps the row's best 64
// candidates sorted in its registers, merges what the streaming waves find as they find
// it, and publishes the k-th best so far as a threshold for them. When the last streaming
// wave is done, only the candidates of its last batches remain to merge before the draw,
// so little of the row's fixed work is left after its last byte arrives.
//
//  Set-up: the row's history ids are loaded first, then the first batch of logits of every
//     streaming wave; the LDS is cleared and one barrier passed. While the first batch is
//     in flight the history ids fill an LDS bitmap of the chunk's history ids (and, for a
//     frequency penalty, a table of the repeated ids and their counts); the streaming
//     waves wait until all of them are in. Once the first batch has been sampled the next
//     two are requested.
//  A. Threshold: every streaming wave adds, for each lane, the final z (penalised if it
//     is a history id) of the lane's largest value in its first batch to an LDS histogram
//     of 12-bit order-key prefixes, and takes the lower edge of the bin that holds the
//     k-th largest value added so far: these are values of distinct ids, so the k-th
//     largest of them bounds the row's k-th best from below. Thresholds taken from raw
//     values elsewhere (masked batches that overflow the stage) are recorded and checked
//     at the end: if the k-th best candidate is at or above the highest of them, nothing
//     in the top k was skipped; otherwise the row is solved exactly (row_solver.hpp; a
//     min-p band that the list cannot hold, band_solver.hpp).
//  B. Stream: raw logits are compared with the raw image of the threshold (x >= thr * T
//     lowered by a margin is implied by z = x * (1/T) >= thr); the slots that pass are
//     compacted into a per-wave LDS stage with ballots, then tempered, penalised if they
//     are history ids, checked against the chunk end and NaN / +inf 64 at a time, and
//     those at or above the threshold are queued for the finisher (an LDS ring). Every
//     queued candidate's final z also goes into a second histogram, whose k-th largest
//     is an exact lower bound of the row's k-th best, read with the sample before each
//     batch; a wave whose batch yields more than k candidates takes their k-th best as
//     its threshold too.
//  C. Finisher: takes queued candidates 64 at a time (one bitonic sort and one bitonic
//     merge into its list, or single insertions for a few) and publishes the k-th best z,
//     an exact lower bound of the row's k-th best, which the streaming waves read before
//     each batch. After the last streaming wave it draws in fp64 (topk_path.hpp), or
//     publishes the chunk's list for topk_finish_kernel.
//
// Min-p as the only filter (band rows): the kept set is every id with z >= zmax +
// ln(min_p), so the thresholds are edges of that band instead of k-th bests: the largest
// final z sampled or queued so far (an LDS maximum), plus ln(min_p) lowered by a margin.
// The finisher keeps the 64 best in its list; a row finished here spills to LDS what leaves
// the list while it is still inside the band of the best z then known (up to kTkSpill
// entries), and when the final band reaches into the spill the whole workgroup draws over
// list and spill (draw_band_candidates). A spill that overflows, or a split row whose list
// cannot hold its band, goes to the band solver's pass over the row.
//
// History ids: when no penalty can raise a logit (repetition >= 1, frequency and presence
// >= 0) an id's penalised z is at most its raw z, so the raw test is enough and history
// ids are penalised when they pass it. Otherwise they are dropped from the stream and the
// row's first chunk scores every history id from the table at the end.
#pragma once

#include "args.hpp"
#include "band_solver.hpp"
#include "block_ops.hpp"
#include "row_solver.hpp"
#include "topk_path.hpp"

namespace arbor {

constexpr int kTkWaves = 16;
constexpr int kTkBlock = kTkWaves * kWave;  // 1024 threads
constexpr int kTkStream = kTkWaves - 1;     // streaming waves; the last wave is the finisher
constexpr int kTkStage = 128;               // raw candidates of one batch staged per wave
constexpr int kTkQueue = 1024;              // candidate ring between the streamers and the finisher
constexpr int kSampleBits = 12;             // threshold histogram: top 12 bits of the order key
constexpr int kSampleBins = 1 << kSampleBits;
constexpr int kTkSpill = 960;               // min-p band entries the finisher may spill (+ 64 in its list)
constexpr int kTkUnitList = 8192;           // masked fp32 rows: listed units with an allowed id (16-bit)
constexpr int kBufferWord3 = 0x00020000;    // buffer resource word 3 (gfx9 family: 32-bit data format)
constexpr int kBufferNt = 2;                // buffer load cache policy: non-temporal
static_assert((kTkQueue & (kTkQueue - 1)) == 0, "the ring size is a power of two");

// 16-byte loads per lane per batch (three batches per lane in flight or in hand), chosen
// by measurement: fp32 2; bf16 3 (min-p band rows of 152K ids: 39.8 us per 512 rows
// against 50.1 with 2 and 43.1 with 1; 4 spills); masked bf16 rows 2 (3 measured slower),
// and unaligned bf16 rows 2 (3 spills there)
#ifndef TK_UNITS_F32
#define TK_UNITS_F32 2
#endif
// Short unmasked aligned rows (WHOLE): one workgroup per row, every wave requests all
// three batches of its ring (three 16-byte units per lane each) at the start, so the row's
// selection waits for one memory latency instead of one per round of the ring; rows of up
// to kTkStream * 64 * 9 units (34,560 fp32 or 69,120 bf16 ids).
constexpr int kTkWholeUnits = 3;
__host__ __device__ constexpr int tk_whole_max_ids(int vec) { return kTkStream * kWave * 3 * kTkWholeUnits * vec; }
template <int DT, bool MASK, bool ALIGNED>
struct TkUnits {
  static constexpr int value = DT == ARBOR_DTYPE_F32 ? TK_UNITS_F32 : (MASK || !ALIGNED ? 2 : 3);
};

// Counts of the sample's lane-maximum keys by their top 12 bits, with a 64-bin summary
// (64 bins each), so that the bin of the k-th largest is found with two wave scans.
struct SampleHist {
  uint32_t fine[kSampleBins];
  uint32_t coarse[kSampleBins / kWave];
};
__device__ __forceinline__ void sample_add(SampleHist& h, uint32_t key) {
  atomicAdd(&h.fine[key >> (32 - kSampleBits)], 1u);
  atomicAdd(&h.coarse[key >> (32 - kSampleBits + 6)], 1u);
}
// Lower edge (as z) of the bin holding the k-th largest key counted so far, or -FLT_MAX
// when fewer than k keys have been counted or the edge is at or below -FLT_MAX. The
// histogram may be read while other waves are still adding to it. Every lane gets it.
__device__ __forceinline__ float sample_threshold(const SampleHist& h, uint32_t k) {
  static_assert(kSampleBins / kWave == kWave, "one summary bin per lane");
  const int lane = lane_id();
  const uint32_t cc = h.coarse[kWave - 1 - lane];  // lane l: l-th highest summary bin
  const uint32_t ci = wave_scan_incl(cc);
  const uint64_t hit = __ballot(ci >= k);
  if (!hit) return -FLT_MAX;
  const int lc = __ffsll((long long)hit) - 1;
  const uint32_t base = lane_get(ci - cc, lc);
  const int cbin = kWave - 1 - lc;
  const uint32_t cf = h.fine[cbin * kWave + kWave - 1 - lane];
  const uint32_t fi = wave_scan_incl(cf);
  const int lf = __ffsll((long long)__ballot(base + fi >= k)) - 1;
  const uint32_t bin = (uint32_t)(cbin * kWave + kWave - 1 - lf);
  return fmaxf(key_value(bin << (32 - kSampleBits)), -FLT_MAX);  // NaN edge (below -inf) -> -FLT_MAX
}

// The k-th largest of the lanes' order keys (0 = none), given at least k nonzero keys:
// the largest prefix with at least k keys at or above it, found bit by bit with ballots.
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t key, int k) {
  // the bits above the highest one where the nonzero keys differ are common to all of
  // them; below it, 16 bits are decided (stopping early leaves a smaller prefix that at
  // least k keys still reach: a lower bound of the k-th largest, which is what the
  // thresholds need)
  const uint32_t hi = wave_max(key);
  const uint32_t lo = wave_min(key != 0u ? key : 0xFFFFFFFFu);
  const uint32_t diff = hi ^ (lo <= hi ? lo : hi);
  if (diff == 0u) return hi;  // every nonzero key is the same (k of them are given)
  const int top = 31 - __builtin_clz(diff);
  uint32_t pre = top == 31 ? 0u : hi & ~((2u << top) - 1u);
  const int stop = top >= 16 ? top - 16 : -1;
  for (int bit = top; bit > stop; --bit) {
    const uint32_t cnd = pre | (1u << bit);
    if (__popcll(__ballot(key >= cnd)) >= k) pre = cnd;
  }
  return pre;
}

struct TkShared {
  uint32_t flags;
  uint32_t tmax;      // order key of the highest sample threshold any wave used
  int hready;         // streaming waves whose history ids are in the bitmap and the table
  int done;           // streaming waves that have queued their last candidate
  uint32_t q_tail;    // candidate slots reserved in the ring
  uint32_t q_head;    // candidate slots the finisher has taken
  uint32_t fin_thr;   // bits of the finisher's k-th best z (-FLT_MAX until it holds k)
  int verdict;        // 1: the finisher's list is exact; 0: the row is solved exactly;
                      // 2: a min-p band row drawn over its list and its spilled entries
  uint32_t band_top;  // min-p band rows: order key of the list's top (0: none)
  uint32_t qtop;      // min-p band rows: order key of the largest final z sampled or queued
  int spill_n;        // min-p band rows drawn over list and spill: entries in `spill`
  uint64_t queue[kTkQueue];
  SampleHist hist;    // lane maxima of every streaming wave's first batch
  union {
    SampleHist chist;  // final z of every queued candidate
    // min-p band rows, which use no candidate histogram: candidates the finisher's list
    // dropped while they were still inside the band of the best z then known
    uint64_t spill[kTkSpill + kWave];
  };
};

// Dynamic LDS of topk_kernel: staged raw candidates | chunk bitmap | history table;
// the row solver's scratch overlays the stages on fallback.
struct TkLds {
  uint64_t* stage;   // [kTkStream * kTkStage]
  uint32_t* bitmap;  // [bitmap_words]
  uint32_t* htab;    // [hash_slots]
  __host__ __device__ static size_t bytes(int bitmap_words, int hash_slots) {
    return sizeof(uint64_t) * kTkStream * kTkStage + sizeof(uint32_t) * ((size_t)bitmap_words + (size_t)hash_slots);
  }
  __device__ TkLds(unsigned char* base, int bitmap_words) {
    stage = reinterpret_cast<uint64_t*>(base);
    bitmap = reinterpret_cast<uint32_t*>(stage + kTkStream * kTkStage);
    htab = bitmap + bitmap_words;
  }
};
static_assert(sizeof(SolverShared) <= sizeof(uint64_t) * kTkStream * kTkStage, "solver scratch fits the stages");
static_assert(band_draw_lds_bytes<kTkBlock>() <= sizeof(uint64_t) * kTkStream * kTkStage,
              "the band draw's scratch fits the stages");
static_assert(kTkSpill + kWave <= kTkBlock, "a band draw takes one candidate per thread");
static_assert(band_lds_bytes(kMaxChunkLen, kTkBlock) <= sizeof(uint64_t) * kTkStream * kTkStage,
              "the band solver's scratch of a whole-row chunk fits the stages");

template <int DT, bool PEN, bool MASK, bool INLINE, bool ALIGNED, bool BAND, bool WHOLE = false>
__global__ void __launch_bounds__(kTkBlock) topk_kernel(Args a) {
  static_assert(!WHOLE || (INLINE && ALIGNED && !MASK), "whole rows: unmasked, aligned, finished here");
  // Every kernel argument the stream uses is read at entry: a scalar load of the argument
  // segment issued later would be one more memory round trip while the first batches are
  // in flight (the compiler otherwise loads them where they are first used).
  __asm__ volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.hist), "s"(a.H), "s"(a.mask), "s"(a.mask_words),
                   "s"(a.uniforms), "s"(a.inv_t), "s"(a.temp), "s"(a.top_k), "s"(a.S), "s"(a.chunk_len),
                   "s"(a.hash_bits), "s"(a.bitmap_words), "s"(a.mask_lds), "s"(a.write_probs), "s"(a.pen_mono), "s"(a.top_p),
                   "s"(a.min_p), "s"(a.out_ids), "s"(a.out_probs));
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int U = WHOLE ? kTkWholeUnits : TkUnits<DT, MASK, ALIGNED>::value;
  constexpr int NQ = VEC * U;        // elements per lane per batch
  constexpr int kBatch = U * kWave;  // units per batch
  constexpr int HIDR = ARBOR_HISTORY_MAX / (kTkStream * kWave) + 1;  // history ids per streaming lane
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ TkShared s;
  const bool hist_inline = PEN && a.pen_mono;
  const bool own_hist = PEN && !hist_inline && (blockIdx.x % a.S) == 0;
  // occurrence counts matter only to a frequency penalty; without one, the bitmap says all
  const bool counts = a.pen.fp != 0.0f;
  const bool table = own_hist || (hist_inline && counts);
  // scored inline, the table needs only the repeats: an id's first occurrence sets its
  // bitmap bit, later ones go to the table (count = 1 + repeats)
  const bool repeats_only = hist_inline && counts;
  TkLds L(smem, PEN ? a.bitmap_words : 0);
  // occurrences of a history id (one whose bitmap bit is set)
  auto count_of = [&](int id) -> uint32_t {
    if (!counts) return 1u;
    const uint32_t n = hist_count(L.htab, (uint32_t)a.hash_bits, (uint32_t)id);
    return repeats_only ? 1u + n : n;
  };

  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;
  const bool finisher = wave == kTkStream;
  const int row = blockIdx.x / a.S, chunk = blockIdx.x % a.S;
  const int c0 = chunk * a.chunk_len;
  const int c1 = min(a.V, c0 + a.chunk_len);
  const void* xrow = row_ptr<DT>(a, row);
  const uint32_t* mrow = MASK ? a.mask + (size_t)row * (size_t)a.mask_words : nullptr;
  const int n_units = (c1 - c0 + VEC - 1) / VEC;
  int n_batches = (n_units + kBatch - 1) / kBatch;  // masked fp32 rows with a unit list: fewer
  // BAND: min-p as the only filter (top_k 0); the list is the whole 64 entries, and it
  // must hold every id of the band z >= zmax + ln(min_p); ln_lo is that bound's
  // safety-margined log
  constexpr bool band = BAND;
  // band rows finished here: entries the list drops inside the band go to an LDS spill
  constexpr bool SPILL = BAND && INLINE;
  const int k = band ? kWave : a.top_k;
  const float ln_lo = a.ln_min_p_lo;

  struct Batch {
    uint32_t w[U][4];  // raw 16-byte units
    uint32_t mw[U];    // mask word of each unit
    int un[U];         // masked fp32 rows: the chunk's unit number of each slot
  };
  // Aligned rows are read with range-checked buffer loads over the chunk: every lane
  // issues one 16-byte load per unit, and a unit past the chunk reads as zeros without a
  // memory access (it is ignored), so the loads in flight stay countable and the ones
  // issued past the end cost no memory round trip.
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(xrow) + (size_t)c0 * Elem<DT>::kBytes), (short)0,
      (c1 - c0) * Elem<DT>::kBytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t mrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(MASK ? mrow : nullptr), (short)0,
                                        MASK ? a.mask_words * 4 : 0, kBufferWord3);
  // Masked fp32 rows: the chunk's mask words are copied to LDS while the first batch is in
  // flight; every later batch reads a unit's word there first and does not request the
  // logits of a unit with no allowed id (a masked logit is -inf whatever its value). bf16
  // rows load each unit's word beside its logits (measured faster for them).
  constexpr bool SKIP = MASK && DT == ARBOR_DTYPE_F32;
  const uint32_t* lmask = SKIP ? reinterpret_cast<const uint32_t*>(smem + a.mask_lds) : nullptr;
  // Their batches after the first ones visit only the units that hold an allowed id: the
  // first batches read the chunk's first kTkStream * kBatch units in order, and later ones
  // take the rest from a list of those units (LDS, after the mask words), built while the
  // first batch is in flight; a chunk with more of them than the list holds walks every
  // unit (n_list < 0).
  const uint16_t* ulist = SKIP ? reinterpret_cast<const uint16_t*>(smem + a.mask_lds + 4 * (a.chunk_len / 32)) : nullptr;
  int n_list = -1;
  constexpr uint32_t kUnitBits = (1u << VEC) - 1u;
  constexpr int kPastChunk = 0x7FFFFFF0;  // a buffer offset past every chunk: reads zeros, no access
  // from_lds: the mask words are in LDS (every batch after the first)
  auto load = [&](int bi, Batch& bt, bool from_lds) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int unit = bi * kBatch + u * kWave + lane;
      if (SKIP && from_lds && n_list >= 0 && bi >= kTkStream) {
        const int li = unit - kTkStream * kBatch;
        unit = li < n_list ? (int)ulist[li] : n_units;
      }
      if (SKIP) bt.un[u] = unit;
      uint32_t mw = 0u;
      bool skip = false;
      if (SKIP && from_lds) {
        mw = unit < n_units ? lmask[(unit * VEC) >> 5] : 0u;
        skip = ((mw >> ((unit * VEC) & 31)) & kUnitBits) == 0u;
      }
      if (ALIGNED) {
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, skip ? kPastChunk : unit * 16, 0, kBufferNt);
        bt.w[u][0] = v.x;
        bt.w[u][1] = v.y;
        bt.w[u][2] = v.z;
        bt.w[u][3] = v.w;
        if (MASK && !(SKIP && from_lds)) mw = __builtin_amdgcn_raw_buffer_load_b32(mrs, ((c0 + unit * VEC) >> 5) * 4, 0, 0);
      } else {
        const int e0 = c0 + unit * VEC;
        if (skip) {
#pragma unroll
          for (int j = 0; j < 4; ++j) bt.w[u][j] = 0u;
        } else {
          load_raw<DT>(xrow, e0, c1, false, bt.w[u]);
        }
        if (MASK && !(SKIP && from_lds)) mw = e0 < c1 ? mrow[e0 >> 5] : 0u;
      }
      if (MASK) bt.mw[u] = mw;
    }
  };
  auto unit_of = [&](int b, const Batch& bt, int q) -> int {
    if constexpr (SKIP) return bt.un[q / VEC];
    return b * kBatch + (q / VEC) * kWave + lane;
  };
  auto id_of = [&](int b, const Batch& bt, int q) { return c0 + unit_of(b, bt, q) * VEC + (q % VEC); };
  // element q of a batch is past the chunk or masked (mw: its unit's mask word)
  // (dropped_u: the same for a slot of unit `unit`)
  auto dropped_u = [&](int unit, int q, uint32_t mw) -> bool {
    if (unit >= n_units) return true;
    if (!ALIGNED && c0 + unit * VEC + (q % VEC) >= c1) return true;
    return MASK && !((mw >> (((c0 + unit * VEC) & 31) + (q % VEC))) & 1u);
  };
  auto dropped_w = [&](int b, const Batch& bt, int q, uint32_t mw) -> bool {
    return dropped_u(unit_of(b, bt, q), q, mw);
  };
  // tempered logit of slot q for the threshold sample: ids past the chunk, masked ids and
  // NaN / +inf read as -inf
  auto zsample = [&](int b, const Batch& bt, int q) __attribute__((always_inline)) -> float {
    if (dropped_w(b, bt, q, MASK ? bt.mw[q / VEC] : 0u)) return -INFINITY;
    const float v = unpack_unit<DT>(bt.w[q / VEC], q % VEC) * a.inv_t;
    return is_invalid(v) ? -INFINITY : v;
  };

  // ---- set-up: the history ids (rows of kTkStream * 64 ids; every streaming lane of
  // such a row loads, clamped, and validity is tested where they are used), the row's
  // uniform and the first batch of every streaming wave; the LDS is cleared and one
  // barrier passed. The first batch is the threshold sample; the next two batches are
  // requested only once it is taken (waves that issue more loads than the memory queue
  // holds stall at the issue and would take the sample late), and the history ids go
  // into the LDS table after that, when they have long arrived ----
  int32_t hraw[HIDR];
  if (PEN) {
    const int32_t* h = a.hist + (size_t)row * (size_t)a.H;
    const int ts = finisher ? 0 : t;
#pragma unroll
    for (int r = 0; r < HIDR; ++r) {
      hraw[r] = -1;
      if (r * kTkStream * kWave < a.H) {
        const int j = ts + r * kTkStream * kWave;
        hraw[r] = h[j < a.H ? j : a.H - 1];
      }
    }
  }
  float u_row = 0.0f;
  if (INLINE) {
    // a vector load (lane-varying zero offset): a scalar one would be waited for by the
    // first LDS wait, long before the value is needed
    int zero;
    __asm__ volatile("v_mov_b32 %0, 0" : "=v"(zero));
    u_row = a.uniforms[row + zero];
  }
  // every wave issues the first batch (no branch around the loads: the compiler would
  // wait for them at the join); the finisher's is past the chunk, which the range-checked
  // loads return as zeros without a memory access
  Batch ba, bb, bc;
  int ia = finisher ? n_batches : wave, ib = wave + kTkStream, ic = wave + 2 * kTkStream;
  load(ia, ba, false);
  if constexpr (WHOLE) {  // the rest of the wave's share (past the chunk: zeros, no access)
    load(ib, bb, false);
    load(ic, bc, false);
  }
  if (SKIP) {
    uint32_t* lm = reinterpret_cast<uint32_t*>(smem + a.mask_lds);
    for (int i = t; i < (c1 - c0 + 31) / 32; i += kTkBlock) lm[i] = mrow[(c0 >> 5) + i];
  }
  if (t == 0) {
    s.flags = 0u;
    s.tmax = 0u;
    s.hready = 0;
    s.done = 0;
    s.q_tail = 0u;
    s.q_head = 0u;
    s.fin_thr = __float_as_uint(-FLT_MAX);
    s.verdict = 1;
    s.qtop = 0u;
  }
  for (int i = t; i < kTkQueue; i += kTkBlock) s.queue[i] = 0ull;
  for (int i = t; i < (int)(sizeof(s.hist) / 4); i += kTkBlock) {
    reinterpret_cast<uint32_t*>(&s.hist)[i] = 0u;
    reinterpret_cast<uint32_t*>(&s.chist)[i] = 0u;
  }
  if (PEN) {
    for (int i = t; i < a.bitmap_words; i += kTkBlock) L.bitmap[i] = 0u;
    if (table)
      for (int i = t; i < (1 << a.hash_bits); i += kTkBlock) L.htab[i] = kEmptySlot;
  }
  __syncthreads();
  if constexpr (SKIP) {
    constexpr int U0 = kTkStream * kBatch;  // units of the first batches
    static_assert(U0 * VEC % 32 == 0, "the first batches end on a mask word");
    if (n_units > U0) {
      // bit j: unit 8 w + j (VEC = 4 ids per unit) is in the chunk and holds an allowed id
      auto unit_bits = [&](int w) -> uint32_t {
        uint32_t nz = lmask[w];
        nz |= nz >> 1;
        nz |= nz >> 2;
        uint32_t bits = 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) bits |= ((nz >> (4 * j)) & 1u) << j;
        const int in_chunk = n_units - 8 * w;
        return in_chunk >= 8 ? bits : bits & ((1u << in_chunk) - 1u);
      };
      // each thread lists the units of a run of mask words, at its place in the block's scan
      const int w0 = U0 * VEC / 32, w1 = (n_units * VEC + 31) / 32;
      const int per = (w1 - w0 + kTkBlock - 1) / kTkBlock;
      const int wa = w0 + t * per, wb = min(w1, wa + per);
      int cnt = 0;
      for (int w = wa; w < wb; ++w) cnt += __popc(unit_bits(w));
      __shared__ int s_scan[kTkWaves];
      int total;
      const int base = block_scan_excl<kTkBlock, int>(cnt, s_scan, &total);
      if (total <= kTkUnitList) {
        uint16_t* ul = const_cast<uint16_t*>(ulist);
        int p = base;
        for (int w = wa; w < wb; ++w) {
          uint32_t bits = unit_bits(w);
          while (bits) {
            ul[p++] = (uint16_t)(8 * w + __builtin_ctz(bits));
            bits &= bits - 1u;
          }
        }
        n_list = total;
        n_batches = kTkStream + (total + kBatch - 1) / kBatch;
      }
      __syncthreads();
    }
  }
  if (a.write_probs) {
    float* prow = a.out_probs + (size_t)row * (size_t)a.V;
    for (int i = c0 + t; i < c1; i += kTkBlock) prow[i] = 0.0f;
  }

  uint64_t best = 0ull;  // the finisher's list: the chunk's best 64 candidates, lane i = i-th
  uint32_t flags = 0u;
  bool exact = false;  // the finisher's verdict: the row is not drawn from its list alone
  if (finisher) {
    // ---- C. the finisher ----
    uint32_t head = 0u;
    float pub = -FLT_MAX;
    int nsp = 0;  // entries spilled (more than kTkSpill: the spill overflowed)
    // the lanes' entries (0: none) at or above `edge` go to the spill
    auto spill = [&](uint64_t d, float edge) {
      const bool sp = d != 0ull && composite_z(d) >= edge;
      const uint64_t m = __ballot(sp);
      if (!m) return;
      const int p = nsp + lanes_below(m);
      if (sp && p < kTkSpill) s.spill[p] = d;
      nsp += __popcll(m);
    };
    for (;;) {
      const uint32_t tail = __atomic_load_n(&s.q_tail, __ATOMIC_RELAXED);
      if (tail == head) {
        // every streaming wave reserves its last slots before it counts itself done
        if (__atomic_load_n(&s.done, __ATOMIC_RELAXED) == kTkStream &&
            __atomic_load_n(&s.q_tail, __ATOMIC_RELAXED) == head)
          break;
        __builtin_amdgcn_s_sleep(1);
        continue;
      }
      const int m = (int)min(tail - head, (uint32_t)kWave);
      const uint32_t slot = (head + (uint32_t)lane) & (kTkQueue - 1);
      uint64_t c = 0ull;
      if (lane < m) {
        // a reserved slot is written by its streaming wave right after the reservation
        c = __atomic_load_n(&s.queue[slot], __ATOMIC_RELAXED);
        while (c == 0ull) {
          __builtin_amdgcn_s_sleep(1);
          c = __atomic_load_n(&s.queue[slot], __ATOMIC_RELAXED);
        }
        s.queue[slot] = 0ull;
      }
      head += (uint32_t)m;
      wave_lds_sync();
      if (lane == 0) __atomic_store_n(&s.q_head, head, __ATOMIC_RELAXED);
      // entries below the list's k-th cannot enter the top k (the streaming waves see the
      // k-th late); the rest are inserted one by one when few, else sorted and merged.
      // Band rows drawn here keep what leaves the list while it is inside the band of the
      // best z so far (lane i of `out`: the i-th entry pushed out by an insertion, or the
      // merge's lower half; `c` where it did not enter).
      {
        const uint64_t kth0 = lane_get(best, k - 1);
        const bool keep = c != 0ull && c > kth0;
        const uint64_t km = __ballot(keep);
        const int nk = __popcll(km);
        uint64_t out = 0ull;
        if (nk > 0 && nk <= 16) {
          uint64_t rest = km;
          int nout = 0;
          while (rest) {
            const int src = __ffsll((long long)rest) - 1;
            rest &= rest - 1;
            const uint64_t ci = lane_get(c, src);
            if (SPILL) {
              // the list's last entry leaves it, or the candidate itself when earlier ones
              // of this batch have lifted the last above it
              const uint64_t last = lane_get(best, kWave - 1);
              if (lane == nout) out = ci > last ? last : ci;
              ++nout;
            }
            best = list_insert(best, ci);
          }
        } else if (nk > 16) {
          const uint64_t srt = wave_sort64_desc(keep ? c : 0ull);
          if (SPILL) {
            const uint64_t rs = lane_reverse(srt);
            out = best < rs ? best : rs;  // the 64 smallest of list and batch
          }
          best = list_merge(best, srt);
        }
        if (SPILL) {
          const float edge = composite_z(lane_get(best, 0)) + ln_lo;
          spill(out, edge);
          spill(keep ? 0ull : c, edge);
        }
      }
      // the k-th best is a lower bound of what is kept (band rows: the queue's top bounds
      // the band's edge, which the streaming waves track themselves)
      const uint64_t kth = lane_get(best, k - 1);
      if (!band && kth != 0ull) {
        const float kz = composite_z(kth);
        if (kz > pub) {
          pub = kz;
          if (lane == 0) __atomic_store_n(&s.fin_thr, __float_as_uint(kz), __ATOMIC_RELAXED);
        }
      }
    }
    wave_lds_sync();
    flags = s.flags;
    // Every candidate passed every threshold its wave used; thresholds from the sample are
    // lower bounds of the k-th best unless history ids in the sample made them overshoot.
    // If the k-th best candidate is at or above the highest of them, nothing in the top k
    // was skipped. Otherwise the row is solved exactly.
    const uint32_t tm = s.tmax;
    bool spilled = false;  // a band row whose band reaches into the spill
    if constexpr (band) {
      // the band's lower edge; a full list whose last entry is still inside it may have
      // dropped members of the band (rows drawn here: those are in the spill, unless it
      // overflowed)
      const uint64_t top = lane_get(best, 0);
      const float edge = composite_z(top) + ln_lo;
      if (tm != 0u && (top == 0ull || order_key(edge) < tm)) flags |= kFlagOverflow;
      if constexpr (SPILL) {
        if (nsp > kTkSpill) {
          flags |= kFlagOverflow;
        } else {
          bool in = false;
          for (int i = lane; i < nsp; i += kWave) in |= composite_z(s.spill[i]) >= edge;
          spilled = __ballot(in) != 0ull;
        }
      } else {
        const uint64_t last = lane_get(best, kWave - 1);
        if (last != 0ull && composite_z(last) >= edge) flags |= kFlagOverflow;
      }
    } else if (tm != 0u) {
      const uint64_t kth = lane_get(best, k - 1);
      if (kth == 0ull || (uint32_t)(kth >> 32) < tm) flags |= kFlagOverflow;
    }
    exact = (flags & kFlagOverflow) && !(flags & (kFlagBadHistory | kFlagInvalid));
    if (exact && lane == 0) {
      s.verdict = 0;
      if constexpr (band) s.band_top = (uint32_t)(lane_get(best, 0) >> 32);  // 0: an empty list
    }
    if (SPILL && !(flags & (kFlagOverflow | kFlagBadHistory | kFlagInvalid)) && spilled) {
      // the whole workgroup draws over the list and the spill after the closing barrier
      const int nl = list_count(best);
      if (lane < nl) s.spill[nsp + lane] = best;
      if (lane == 0) {
        s.verdict = 2;
        s.spill_n = nsp + nl;
        s.band_top = (uint32_t)(lane_get(best, 0) >> 32);
      }
      exact = true;  // the list alone is not the answer
    }
  } else {
    // ---- A. the history ids go into the bitmap (and the count table) while the first
    // batch is in flight; once every streaming wave's are in, the final z of each lane's
    // largest value in its first batch joins the sample. These are values of distinct ids,
    // so the k-th largest of the sample bounds the row's k-th best from below even when
    // the largest logits are history ids that a penalty lowers (as in a generation loop,
    // whose history holds the tokens just sampled). Then the next two batches are
    // requested ----
    if (PEN) {
      bool badh = false;
#pragma unroll
      for (int r = 0; r < HIDR; ++r) {
        const int32_t id = t + r * kTkStream * kWave < a.H ? hraw[r] : -1;
        if (id >= a.V) {
          badh = true;
        } else if (id >= 0) {
          const bool in_chunk = id >= c0 && id < c1;
          const uint32_t bit = 1u << ((id - c0) & 31);
          if (repeats_only) {
            if (in_chunk && (atomicOr(&L.bitmap[(id - c0) >> 5], bit) & bit))
              hist_insert(L.htab, (uint32_t)a.hash_bits, (uint32_t)id);
          } else {
            if (in_chunk) atomicOr(&L.bitmap[(id - c0) >> 5], bit);
            if (table) hist_insert(L.htab, (uint32_t)a.hash_bits, (uint32_t)id);
          }
        }
      }
      if (__ballot(badh) && lane == 0) atomicOr(&s.flags, kFlagBadHistory);
      wave_lds_sync();
      if (lane == 0) {
        atomicAdd(&s.hready, 1);
        // every streaming wave inserts before it waits, and none queues anything before
        while (__atomic_load_n(&s.hready, __ATOMIC_RELAXED) < kTkStream) __builtin_amdgcn_s_sleep(1);
      }
      wave_lds_sync();
    }
    {
      float lm = -INFINITY;
      int lid = 0;  // its id
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const float v = zsample(ia, ba, q);
        if (v > lm) {
          lm = v;
          lid = id_of(ia, ba, q);
        }
      }
      if (PEN && lm > -INFINITY) {
        // as in the stream: a history id is penalised, or (when a penalty may raise it, and
        // the row's first chunk scores every history id at the end) left out
        const int id = lid, off = id - c0;
        if ((L.bitmap[off >> 5] >> (off & 31)) & 1u)
          lm = hist_inline ? penalize(lm, count_of(id), a.pen) : -INFINITY;
      }
      if constexpr (band) {
        // band rows take the sample's largest, the final z of a real id, as a lower bound
        // of zmax (and the threshold its band's edge)
        const uint32_t km = wave_max(order_key(lm + 0.0f));
        if (lane == 0) atomicMax(&s.qtop, km);
      } else {
        sample_add(s.hist, order_key(lm + 0.0f));
      }
      wave_lds_sync();
    }
    if constexpr (!WHOLE) {
      load(ib, bb, true);
      load(ic, bc, true);
    }

    // ---- B. stream ----
    uint64_t* stage = L.stage + wave * kTkStage;
    bool bad = false;
    // z >= thr is accepted; x >= x_thr is implied by z = fl(x * (1/T)) >= thr
    float thr = 0.0f, x_thr = 0.0f;
    auto set_thr = [&](float tv) {
      thr = uniform(tv);
      const float tt = thr * a.temp;
      x_thr = uniform(tt - (fabsf(tt) * 0x1p-20f + 0x1p-120f));
    };
    // thresholds read from the sample histogram are recorded (checked at the end); those
    // from the candidate histogram (the k-th best queued so far, to a 12-bit bin edge) and
    // the finisher's k-th best are exact lower bounds
    uint32_t tmax_w = 0u;
    auto refresh = [&]() {
      if constexpr (band) {
        // the band's edge below the largest final z sampled or queued so far: every member
        // of the band passes it
        const uint32_t qt = __atomic_load_n(&s.qtop, __ATOMIC_RELAXED);
        const float tn = qt != 0u ? key_value(qt) + ln_lo : -FLT_MAX;
        if (tn > thr) set_thr(tn);
        return;
      }
      const float ts = sample_threshold(s.hist, (uint32_t)k);
      const float tc = fmaxf(sample_threshold(s.chist, (uint32_t)k),
                             __uint_as_float(__atomic_load_n(&s.fin_thr, __ATOMIC_RELAXED)));
      if (ts > thr && ts > tc) tmax_w = order_key(ts);
      const float tn = fmaxf(ts, tc);
      if (tn > thr) set_thr(tn);
    };
    set_thr(-FLT_MAX);  // the stream loop refreshes before its first batch
    // batches are interleaved over the streaming waves (wave w takes w, w + 15, ...)
    int nextb = wave + 3 * kTkStream;
    auto grab = [&]() -> int {
      const int b = nextb;
      nextb += kTkStream;
      return b;
    };
    // queue the lanes' candidates (final z) for the finisher
    auto emit = [&](bool tk, float v, int id) __attribute__((always_inline)) {
      const uint64_t m = __ballot(tk);
      if (!m) return;
      uint32_t base = 0u;
      uint32_t km = 0u;
      if constexpr (band) km = wave_max(tk ? order_key(v + 0.0f) : 0u);
      if (lane == 0) {
        base = atomicAdd(&s.q_tail, (uint32_t)__popcll(m));
        if (band) atomicMax(&s.qtop, km);
      }
      base = lane_get(base, 0);
      if (tk) {
        const uint32_t p = base + (uint32_t)lanes_below(m);
        // the ring slot is free once the finisher has taken the entry kTkQueue places back
        const uint64_t c = composite(v + 0.0f, id);
        if (!band) sample_add(s.chist, (uint32_t)(c >> 32));
        while (p - __atomic_load_n(&s.q_head, __ATOMIC_RELAXED) >= (uint32_t)kTkQueue) __builtin_amdgcn_s_sleep(1);
        __atomic_store_n(&s.queue[p & (kTkQueue - 1)], c, __ATOMIC_RELAXED);
      }
    };
    // final z of a candidate whose raw logit passed (id inside the chunk, z not NaN / +inf):
    // history ids are penalised, or dropped (-inf) when the row's first chunk scores them
    auto final_z = [&](float v, int id) -> float {
      if (PEN) {
        const int off = id - c0;
        if ((L.bitmap[off >> 5] >> (off & 31)) & 1u)
          v = hist_inline ? penalize(v, count_of(id), a.pen) : -INFINITY;
      }
      return v;
    };
    // raw test of slot q: x >= x_thr, or NaN (flagged when it is looked at)
    auto passes = [&](int b, const Batch& bt, int q) __attribute__((always_inline)) -> bool {
      const float x = unpack_unit<DT>(bt.w[q / VEC], q % VEC);
      bool p = !(x < x_thr);
      if (MASK) p = p && ((bt.mw[q / VEC] >> (((c0 + unit_of(b, bt, q) * VEC) & 31) + (q % VEC))) & 1u);
      return p;
    };
    // one candidate per lane whose raw logit passed. When more than k of the wave's lanes
    // hold one at or above the threshold, the k-th largest of them (final z) is a lower
    // bound of the row's k-th best and becomes the wave's threshold (this bounds what is
    // queued while the threshold is still far below the row's k-th best).
    auto consider = [&](bool tk, float x, int id) __attribute__((always_inline)) {
      float v = -INFINITY;
      if (tk) {
        v = x * a.inv_t;
        if (is_invalid(v)) {
          bad = true;  // NaN, +inf, or overflow to +inf
          tk = false;
        } else {
          v = final_z(v, id);
        }
      }
      tk = tk && v >= thr;
      if constexpr (band) {
        const float vm = wave_max(tk ? v : -FLT_MAX);
        if (vm + ln_lo > thr) {
          set_thr(vm + ln_lo);
          tk = tk && v >= thr;
        }
      } else if (__popcll(__ballot(tk)) > k) {
        set_thr(fmaxf(thr, key_value(wave_kth_key(tk ? order_key(v) : 0u, k))));
        tk = tk && v >= thr;
      }
      emit(tk, v, id);
    };
    // Staged raw candidates (x bits << 32 | id), 64 per round across the lanes.
    auto absorb = [&](int ns) __attribute__((always_inline)) {
#pragma unroll 1
      for (int j = 0; j < ns; j += kWave) {
        const int i = j + lane;
        const uint64_t e = i < ns ? stage[i] : 0ull;
        const int id = (int)(uint32_t)e;
        // ids past the chunk are the zeros read past its end
        consider(i < ns && id < c1, __uint_as_float((uint32_t)(e >> 32)), id);
      }
    };
    auto process = [&](int b, const Batch& bt) __attribute__((always_inline)) {
      // stage the passing slots while the stage has room
      int ns = 0;
      bool full = false;
      auto stage_passing = [&]() __attribute__((always_inline)) {
        ns = 0;
        full = false;
        // masked fp32 rows vote over the whole batch first: most of their batches hold no
        // passing slot, and the slot-by-slot loop below costs a wave-wide branch per slot
        // (in the other instances the vote measured slower than it saves)
        if constexpr (SKIP) {
          bool any = false;
#pragma unroll
          for (int q = 0; q < NQ; ++q) any |= passes(b, bt, q);
          if (!__ballot(any)) return;
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const bool p = passes(b, bt, q);
          const uint64_t m = __ballot(p);
          if (m) {
            const int c = __popcll(m);
            if (ns + c <= kTkStage) {
              if (p)
                stage[ns + lanes_below(m)] =
                    ((uint64_t)__float_as_uint(unpack_unit<DT>(bt.w[q / VEC], q % VEC)) << 32) | (uint32_t)id_of(b, bt, q);
              ns += c;
            } else {
              full = true;
            }
          }
        }
      };
      stage_passing();
      if (MASK && __builtin_expect(full, 0)) {
        // More passing slots than the stage holds (a threshold far below the row's k-th
        // best, as on masked rows, whose masked lanes leave the sample short): the k-th
        // largest of the lanes' best passing z, k distinct ids, bounds the row's k-th best
        // from below (band: the best one bounds zmax). Raw values cannot see penalties, so
        // with history ids the bound is checked at the end like the sample. Rows without a
        // mask rarely get here and keep the code of their stream loop small.
        float lm = -INFINITY;
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          if (passes(b, bt, q) && !dropped_w(b, bt, q, MASK ? bt.mw[q / VEC] : 0u))
            lm = fmaxf(lm, unpack_unit<DT>(bt.w[q / VEC], q % VEC));
        const float zl = lm * a.inv_t + 0.0f;
        const uint32_t key = lm > -INFINITY && !is_invalid(zl) ? order_key(zl) : 0u;
        float tb = -FLT_MAX;
        if (!band && __popcll(__ballot(key != 0u)) >= k) tb = key_value(wave_kth_key(key, k));
        if constexpr (band) {
          const uint32_t km = wave_max(key);
          if (km != 0u) tb = fmaxf(tb, key_value(km) + ln_lo);
        }
        if (tb > thr) {
          if (PEN) tmax_w = max(tmax_w, order_key(tb));
          set_thr(tb);
          stage_passing();
        }
      }
      if (ns == 0 && !full) return;
      if (__builtin_expect(!full, 1)) {
        wave_lds_sync();
        absorb(ns);
      } else {
        // more than the stage holds (a threshold far below the row's k-th best): one slot
        // at a time, picked by selects so that the candidate code exists once
#pragma unroll 1
        for (int q = 0; q < NQ; ++q) {
          float x = 0.0f;
          uint32_t mw = 0u;
          bool p = false;
          int un = 0;
#pragma unroll
          for (int qq = 0; qq < NQ; ++qq) {
            if (qq == q) {
              x = unpack_unit<DT>(bt.w[qq / VEC], qq % VEC);
              mw = MASK ? bt.mw[qq / VEC] : 0u;
              p = passes(b, bt, qq);
              un = unit_of(b, bt, qq);
            }
          }
          if (!__ballot(p)) continue;
          consider(p && !dropped_u(un, q, mw), x, c0 + un * VEC + (q % VEC));
        }
      }
    };
    if constexpr (WHOLE) {
      // the wave's three batches are its whole share of the row
      if (ia < n_batches) {
        refresh();
        process(ia, ba);
      }
      if (ib < n_batches) process(ib, bb);
      if (ic < n_batches) process(ic, bc);
    }
    for (; !WHOLE;) {
      if (ia >= n_batches) break;
      refresh();
      process(ia, ba);
      ia = grab();
      load(ia, ba, true);
      if (ib >= n_batches) break;
      process(ib, bb);
      ib = grab();
      load(ib, bb, true);
      if (ic >= n_batches) break;
      process(ic, bc);
      ic = grab();
      load(ic, bc, true);
    }

    // history ids a penalty may raise: the row's first chunk scores all of them
    if (own_hist) {
      // streaming waves take interleaved 64-slot slices of the table (a power of two >= 64)
      for (int sb = wave; sb * kWave < (1 << a.hash_bits); sb += kTkStream) {
        const int slot = sb * kWave + lane;
        const uint32_t e = L.htab[slot];
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
        emit(z >= thr, z, id);
      }
    }
    const bool wbad = __ballot(bad) != 0ull;  // bad is per lane
    wave_lds_sync();                          // this wave's queue entries are written
    if (lane == 0) {
      if (wbad) atomicOr(&s.flags, kFlagInvalid);
      if (tmax_w) atomicMax(&s.tmax, tmax_w);
    }
    wave_lds_sync();
    if (lane == 0) atomicAdd(&s.done, 1);
  }
  // The finisher draws (or publishes the chunk's list) before the closing barrier, which
  // only the exact solver needs: the streaming waves wait there for the verdict.
  if (finisher && !exact) {
    const int n = min(k, list_count(best));
    if (INLINE) {
      if (flags & kFlagBadHistory) {
        if (lane == 0) a.out_ids[row] = ARBOR_ID_BAD_HISTORY;
      } else if (flags & kFlagInvalid) {
        if (lane == 0) a.out_ids[row] = ARBOR_ID_INVALID;
      } else if (n == 0) {
        if (lane == 0) a.out_ids[row] = ARBOR_ID_EMPTY;
      } else {
        finish_list(a, row, best, n, u_row);
      }
    } else {
      const size_t slot = (size_t)row * (size_t)a.S + (size_t)chunk;
      if (lane < n) a.cand[slot * kChunkSlot + lane] = best;
      if (lane == 0) {
        a.hdr[slot * 2 + 0] = (uint32_t)n;
        a.hdr[slot * 2 + 1] = flags;
      }
    }
  }
  __syncthreads();
  if (SPILL && s.verdict == 2) {
    // every member of the band is in the list or the spill
    draw_band_candidates<kTkBlock>(a, row, s.spill, s.spill_n, s.band_top, u_row,
                                   reinterpret_cast<unsigned char*>(L.stage));
  } else if (s.verdict == 0) {
    if (INLINE && BAND) {
      // a band the list could not hold: one more pass over the row, which is still in the
      // caches, from the list's top (the row's maximum unless candidates were lost)
      solve_band_row<kTkBlock, DT, ALIGNED>(a, row, s.band_top, L.htab, reinterpret_cast<unsigned char*>(L.stage));
    } else if (INLINE) {
      solve_row<kTkBlock, DT>(a, row, L.htab, *reinterpret_cast<SolverShared*>(L.stage));
    } else if (finisher && lane == 0) {
      const size_t slot = (size_t)row * (size_t)a.S + (size_t)chunk;
      a.hdr[slot * 2 + 0] = 0u;
      a.hdr[slot * 2 + 1] = flags;
    }
  }
}

}  // namespace arbor
