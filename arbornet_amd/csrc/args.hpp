// args.hpp -- launch arguments, workload constants and element loads shared by the
// sampling kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/arbor_sampling.h"
#include "device_common.hpp"

namespace arbor {

constexpr int kBlock = 1024;               // threads of every sampling workgroup
constexpr int kWaves = kBlock / kWave;     // 16
constexpr int kChunkSlot = 64;             // candidates one chunk of a split row publishes
constexpr int kMaxTopK = 64;               // largest top-k of the streaming path
constexpr int kMaxChunks = 64;             // chunks a row may be split into
constexpr int kMaxChunkLen = 262144;       // ids per chunk (chunk bitmap <= 32 KB)
constexpr int kMaxHashBits = 13;           // history table slots <= 8192 (H <= 4096)

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
  float temp;  // temperature (raw-logit thresholds)
  Penalty pen;
  int top_k;          // 0 = off (k >= V is off)
  float top_p;        // 1 = off
  float min_p;        // 0 = off
  float ln_min_p_lo;  // ln(min_p) minus a safety margin: the min-p candidate band
  double ln_min_p;    // ln(min_p) in fp64: z is in the band iff (double)z - zmax >= ln_min_p
  int S, chunk_len;
  int hash_bits, bitmap_words;
  int mask_lds;  // masked streamed rows: byte offset of the chunk's allow-mask words in dynamic LDS
  int aligned, write_probs;
  int pen_mono;  // repetition >= 1, frequency >= 0, presence >= 0: a penalty never raises z
  uint32_t* hdr;   // [B*S*2]            count, flags of each chunk list
  uint64_t* cand;  // [B*S*kChunkSlot]   sorted candidate composites of each chunk
  float* zbuf;     // [B*ldz]            row solver's tempered logits
  int ldz;         // zbuf row stride: V rounded up to 64 floats (rows 256-byte aligned)
  // generation step (rows finished by one workgroup): the history ring and its write
  // positions; the thread that writes a row's id also appends it, after the row's history
  // was read
  int32_t* ring_hist;  // == hist, writable; null: no append
  int32_t* ring_pos;   // [B]
};

template <int DT>
struct Elem;
template <>
struct Elem<ARBOR_DTYPE_F32> {
  static constexpr int kVec = 4;
  static constexpr int kBytes = 4;
  static __device__ __forceinline__ float one(const void* base, int64_t i) {
    return static_cast<const float*>(base)[i];
  }
  // streaming 16-byte load: logits are read once, so the load is marked non-temporal
  static __device__ __forceinline__ void vec(const void* base, int64_t i, float* x) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(static_cast<const float*>(base) + i));
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  }
};
template <>
struct Elem<ARBOR_DTYPE_BF16> {
  static constexpr int kVec = 8;
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float one(const void* base, int64_t i) {
    return bf16_bits_to_float(static_cast<const uint16_t*>(base)[i]);
  }
  static __device__ __forceinline__ void vec(const void* base, int64_t i, float* x) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(static_cast<const uint16_t*>(base) + i));
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

// Raw 16-byte unit (VEC elements) starting at e0; positions at or beyond `end` hold -inf.
// Kept raw in registers while in flight and converted by unpack_unit when processed.
template <int DT>
__device__ __forceinline__ void load_raw(const void* row, int e0, int end, bool aligned, uint32_t* w) {
  constexpr int VEC = Elem<DT>::kVec;
  if (aligned && e0 + VEC <= end) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_nontemporal_load(
        reinterpret_cast<const u4*>(static_cast<const char*>(row) + (size_t)e0 * Elem<DT>::kBytes));
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
  } else if (DT == ARBOR_DTYPE_F32) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = e0 + j < end ? static_cast<const uint32_t*>(row)[e0 + j] : 0xFF800000u;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = e0 + 2 * j < end ? static_cast<const uint16_t*>(row)[e0 + 2 * j] : 0xFF80u;
      const uint32_t hi = e0 + 2 * j + 1 < end ? static_cast<const uint16_t*>(row)[e0 + 2 * j + 1] : 0xFF80u;
      w[j] = lo | (hi << 16);
    }
  }
}
template <int DT>
__device__ __forceinline__ float unpack_unit(const uint32_t* w, int j) {
  if (DT == ARBOR_DTYPE_F32) return __uint_as_float(w[j]);
  return __uint_as_float((j & 1) ? (w[j >> 1] & 0xFFFF0000u) : (w[j >> 1] << 16));
}

template <int DT>
__device__ __forceinline__ const void* row_ptr(const Args& a, int row) {
  return static_cast<const char*>(a.logits) + (size_t)row * (size_t)a.ld * (size_t)Elem<DT>::kBytes;
}

// The row's sampled id goes to slot positions[row] mod H of its history ring, and the
// position advances (sentinels append nothing). Penalties count occurrences, so the
// ring's order does not matter. Called by the one thread that writes out_ids[row].
__device__ __forceinline__ void ring_append(const Args& a, int row, int32_t id) {
  if (a.ring_pos == nullptr || id < 0) return;
  const uint32_t pos = (uint32_t)a.ring_pos[row];
  a.ring_hist[(size_t)row * (size_t)a.H + pos % (uint32_t)a.H] = id;
  a.ring_pos[row] = (int32_t)(pos + 1u);
}

}  // namespace arbor
