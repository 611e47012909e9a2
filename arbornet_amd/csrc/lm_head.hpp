// lm_head.hpp -- the step before the sampler: logits = (x · Wᵀ + bias) · scale on the
// gfx950 matrix cores (v_mfma_f32_32x32x16_bf16: bf16 operands, fp32 accumulation), with
// the bias, the scale (1/T when the caller folds the temperature in), an optional bf16
// cast and each row's maximum in the epilogue.
//
// Shapes: x [B, H] (fp32 or bf16, rows ld_x apart), W [V, H] as vocabulary rows, logits
// [B, V] (rows ld_out apart). At decode batches the product is bound by reading W once
// from HBM (2·H·V bytes against 2·B·H·V flops: B = 256 is just below the bf16 ridge of
// 2.5 PFLOP/s over 8 TB/s), so the kernel is organised around that read:
//  - W is packed once, at load time, into the A-operand order of the instruction: for
//    each tile of 32 vocabulary rows and each step of 16 hidden ids, 64 lanes × 16 bytes,
//    lane l holding W[32t + l % 32][16s + 8(l / 32) .. +8]. A wave's operand for one step
//    is then one contiguous 1 KB load, and W is read exactly once, straight into
//    registers, three stages of 32 hidden ids ahead of its use.
//  - x is small and used by every vocabulary row: each workgroup stages chunks of 32
//    hidden ids of all B rows in LDS, already in the B-operand order (lane l of N-tile n
//    holding x[32n + l % 32][16s + 8(l / 32) .. +8]), double-buffered, so each wave reads
//    a fragment as one conflict-free 16-byte LDS load per lane.
//  - A workgroup of 8 waves covers 256 vocabulary rows (32 per wave) and all B ≤ 256 rows
//    (NT = B / 32 N-tiles: 16·NT accumulator registers per lane).
//  - Every load is unconditional (clamped addresses), and the hidden size is a multiple
//    of the four-stage ring (128), so the ring's registers stay fixed across the unrolled
//    stages and the waits before each stage's instructions leave the next stages' loads
//    in flight (conditional loads made the compiler copy the ring and wait for everything:
//    406 -> 363 us).
// Accumulator layout of the 32×32 result (register r of lane l): row i = 8(r / 4) +
// 4(l / 32) + r % 4 (a vocabulary row), column j = l % 32 (a batch row).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/arbor_sampling.h"
#include "device_common.hpp"

namespace arbor {

typedef __bf16 lm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lm_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int lm_u4 __attribute__((ext_vector_type(4)));

constexpr int kLmWaves = 8;
constexpr int kLmThreads = kLmWaves * kWave;  // 512
constexpr int kLmRows = kLmWaves * 32;        // vocabulary rows per workgroup
constexpr int kLmKt = 32;                     // hidden ids per LDS stage
constexpr int kLmBufs = 4;                    // weight stages in registers (three ahead of the one in use)
constexpr int kLmHidden = kLmKt * kLmBufs;     // hidden sizes: multiples of 128
constexpr int kLmSteps = kLmKt / 16;          // MFMA k-steps per stage
constexpr int kLmMaxB = 256;                  // batch rows per launch

// Packed W: vocabulary rows padded to a multiple of kLmRows, zeros beyond V.
__host__ __device__ inline size_t lm_packed_bytes(int H, int V) {
  const size_t rows = ((size_t)V + kLmRows - 1) / kLmRows * kLmRows;
  return rows * (size_t)H * 2u;
}

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint32_t lm_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// One packed 16-byte unit per thread: vocabulary row v, hidden ids h0 .. h0 + 7.
// layout ARBOR_LM_WEIGHT_HV: W given as [H, V] (the reference's Linear.weight, in x out);
// ARBOR_LM_WEIGHT_VH: [V, H].
template <int WDT>
__global__ void __launch_bounds__(256) lm_pack_kernel(const void* w, int layout, int H, int V, int rows,
                                                      lm_u4* packed) {
  const size_t q = (size_t)blockIdx.x * 256u + threadIdx.x;
  if (q >= (size_t)rows * (size_t)(H / 8)) return;
  // thread order: consecutive threads take consecutive vocabulary rows of one hidden group
  // (8 ids), so [H, V] reads are coalesced along V and packed writes along the lanes
  const int hg = (int)(q / (size_t)rows);
  const int v = (int)(q % (size_t)rows);
  const int h0 = hg * 8;
  uint32_t b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float f = 0.0f;
    uint32_t bits = 0u;
    if (v < V) {
      const size_t idx = layout == ARBOR_LM_WEIGHT_HV ? (size_t)(h0 + j) * (size_t)V + (size_t)v
                                                      : (size_t)v * (size_t)H + (size_t)(h0 + j);
      if (WDT == ARBOR_DTYPE_F32) {
        f = static_cast<const float*>(w)[idx];
        bits = lm_bf16_bits(f);
      } else {
        bits = static_cast<const uint16_t*>(w)[idx];
      }
    }
    b[j] = bits;
  }
  const int t = v / 32, s = h0 / 16, lane = (v % 32) + 32 * ((h0 / 8) % 2);
  const size_t unit = ((size_t)t * (size_t)(H / 16) + (size_t)s) * 64u + (size_t)lane;
  lm_u4 o;
  o.x = b[0] | (b[1] << 16);
  o.y = b[2] | (b[3] << 16);
  o.z = b[4] | (b[5] << 16);
  o.w = b[6] | (b[7] << 16);
  packed[unit] = o;
}

struct LmArgs {
  const void* x;
  int64_t ld_x;
  const lm_u4* w;  // packed
  const float* bias;
  void* out;
  int64_t ld_out;
  float* row_max;
  float scale;
  int B, H, V;
};

__global__ void lm_fill_kernel(float* p, int n, float v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// max of two floats through their order (a NaN is never the maximum)
__device__ __forceinline__ void lm_atomic_max(float* p, float v) {
  if (!(v == v)) return;
  unsigned int* u = reinterpret_cast<unsigned int*>(p);
  unsigned int cur = __hip_atomic_load(u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (__uint_as_float(cur) < v || (__uint_as_float(cur) != __uint_as_float(cur))) {
    const unsigned int prev = atomicCAS(u, cur, __float_as_uint(v));
    if (prev == cur) break;
    cur = prev;
  }
}

// The workgroup's waves as WM (vocabulary) x WN (batch): each wave computes MT tiles of 32
// vocabulary rows for NT / WN N-tiles of 32 batch rows, so each x fragment it reads from
// LDS feeds MT instructions (MT = 8 / WM: 256 vocabulary rows per workgroup). Measured at
// B = 256, H = 4096, V = 128256: WN = 1 (every wave loads its own W rows once) 354 us,
// WN = 2 (two waves load the same W rows, each x fragment feeds two instructions) 362 us.
template <int NT>
struct LmGrid {
  static constexpr int WN = 1;
  static constexpr int WM = kLmWaves / WN;
  static constexpr int MT = kLmRows / 32 / WM;
  static constexpr int NTW = NT / WN;
};

// NT: batch N-tiles of 32 rows; XDT: x dtype; ODT: logits dtype
template <int NT, int XDT, int ODT>
__global__ void __launch_bounds__(kLmThreads) lm_head_kernel(LmArgs a) {
  using G = LmGrid<NT>;
  constexpr int MT = G::MT, NTW = G::NTW, WM = G::WM;
  constexpr int kSlots = kLmSteps * NT * kWave;  // 16-byte x fragments per stage
  __shared__ __align__(16) lm_u4 xs[2][kSlots];
  static_assert(sizeof(float) * WM * NT * 32 <= sizeof(lm_u4) * kSlots, "row maxima fit a stage");
  float (*smax)[NT * 32] = reinterpret_cast<float (*)[NT * 32]>(&xs[0][0]);  // after the last stage
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int H = a.H;
  const int tile0 = blockIdx.x * (kLmRows / 32) + wm * MT;  // the wave's first tile of 32 vocabulary rows
  const int n_steps = H / 16, n_chunks = H / kLmKt;
  const lm_u4* wp = a.w + (size_t)tile0 * (size_t)n_steps * 64u + lane;

  // x staging: slot q of a stage <-> batch row b = q / G8, hidden group g = q % G8 (8 ids)
  constexpr int G8 = kLmKt / 8;
  constexpr int kStage = NT * 32 * G8;                            // slots per stage
  constexpr int kPer = (kStage + kLmThreads - 1) / kLmThreads;  // slots per thread
  lm_u4 xr[kLmBufs][kPer];  // x of the next stages, kLmBufs - 1 ahead like W
  auto x_load = [&](int c, lm_u4* xr_) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int q = t + i * kLmThreads;
      // unconditional loads from clamped rows (batch rows past B repeat row B - 1; their
      // products are never stored), so that the loaded registers need no merge with a
      // default and stay in place across the unrolled stages
      const int qc = q < kStage ? q : kStage - 1;
      const int b = min(qc / G8, a.B - 1), g = qc % G8;
      lm_u4 v;
      {
        const size_t off = (size_t)b * (size_t)a.ld_x + (size_t)(c * kLmKt + g * 8);
        if (XDT == ARBOR_DTYPE_BF16) {
          v = *reinterpret_cast<const lm_u4*>(static_cast<const uint16_t*>(a.x) + off);
        } else {
          const float4* f = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + off);
          const float4 f0 = f[0], f1 = f[1];
          v.x = lm_bf16_bits(f0.x) | (lm_bf16_bits(f0.y) << 16);
          v.y = lm_bf16_bits(f0.z) | (lm_bf16_bits(f0.w) << 16);
          v.z = lm_bf16_bits(f1.x) | (lm_bf16_bits(f1.y) << 16);
          v.w = lm_bf16_bits(f1.z) | (lm_bf16_bits(f1.w) << 16);
        }
      }
      xr_[i] = v;
    }
  };
  auto x_store = [&](int buf, const lm_u4* xr_) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int q = t + i * kLmThreads;
      if (q < kStage) {
        const int b = q / G8, g = q % G8;
        const int s = g >> 1, l = (b & 31) + 32 * (g & 1), n = b >> 5;
        xs[buf][(s * NT + n) * kWave + l] = xr_[i];
      }
    }
  };

  lm_f32x16 acc[MT][NTW];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < NTW; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.0f;

  // W: kLmBufs - 1 stages in flight ahead of the one in use
  lm_u4 wr[kLmBufs][MT][kLmSteps];
  auto w_load = [&](int c, lm_u4 (*dst)[kLmSteps]) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int s = 0; s < kLmSteps; ++s)
        dst[m][s] = wp[((size_t)m * (size_t)n_steps + (size_t)(c * kLmSteps + s)) * 64u];
  };
#pragma unroll
  for (int c = 0; c < kLmBufs - 1; ++c) {
    x_load(c, xr[c]);
    w_load(c, wr[c]);
  }
  x_store(0, xr[0]);
  __syncthreads();

  // n_chunks is a multiple of kLmBufs (hidden % 128 == 0), so the ring's slots are fixed
  // registers across the unrolled stages
  for (int c0 = 0; c0 < n_chunks; c0 += kLmBufs) {
#pragma unroll
    for (int u = 0; u < kLmBufs; ++u) {
      const int c = c0 + u;
      const int buf = u & 1;
      // the stage kLmBufs - 1 ahead (clamped: past the end the last stage is requested
      // again, unused): its x and W requests go out now; the x of the next stage
      // (requested kLmBufs - 2 stages ago) goes to LDS at the end of this one
      {
        const int ca = min(c + kLmBufs - 1, n_chunks - 1);
        x_load(ca, xr[(u + kLmBufs - 1) % kLmBufs]);
        w_load(ca, wr[(u + kLmBufs - 1) % kLmBufs]);
      }
#pragma unroll
      for (int s = 0; s < kLmSteps; ++s) {
#pragma unroll
        for (int n = 0; n < NTW; ++n) {
          const lm_bf16x8 bv =
              __builtin_bit_cast(lm_bf16x8, xs[buf][(s * NT + wn * NTW + n) * kWave + lane]);
#pragma unroll
          for (int m = 0; m < MT; ++m)
            acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(lm_bf16x8, wr[u][m][s]), bv,
                                                                acc[m][n], 0, 0, 0);
        }
      }
      x_store(buf ^ 1, xr[(u + 1) % kLmBufs]);  // past the end: written, never read
      __syncthreads();
    }
  }

  // epilogue: bias, scale, cast, store; the row maxima of the stored values
  float mrow[NTW];
#pragma unroll
  for (int n = 0; n < NTW; ++n) mrow[n] = -INFINITY;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int v_base = (tile0 + m) * 32 + 4 * (lane >> 5);
    float bias_r[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = v_base + 8 * (r >> 2) + (r & 3);
      bias_r[r] = (a.bias && v < a.V) ? a.bias[v] : 0.0f;
    }
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
      const int b = (wn * NTW + n) * 32 + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float y = (acc[m][n][4 * g + e] + bias_r[4 * g + e]) * a.scale;
          if (ODT == ARBOR_DTYPE_BF16) y = __uint_as_float(lm_bf16_bits(y) << 16);
          o[e] = y;
        }
        const int v0 = v_base + 8 * g;
        if (b < a.B) {
          if (ODT == ARBOR_DTYPE_F32) {
            float* dst = static_cast<float*>(a.out) + (size_t)b * (size_t)a.ld_out + (size_t)v0;
            if (v0 + 3 < a.V && ((a.ld_out & 3) == 0)) {
              *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (v0 + e < a.V) dst[e] = o[e];
            }
          } else {
            uint16_t* dst = static_cast<uint16_t*>(a.out) + (size_t)b * (size_t)a.ld_out + (size_t)v0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (v0 + e < a.V) dst[e] = (uint16_t)(__float_as_uint(o[e]) >> 16);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (v0 + e < a.V && o[e] > mrow[n]) mrow[n] = o[e];
        }
      }
    }
  }
  // the wave's rows: lanes l and l + 32 hold the same batch row
#pragma unroll
  for (int n = 0; n < NTW; ++n) {
    const float other = __shfl_xor(mrow[n], 32);
    const float m = other > mrow[n] ? other : mrow[n];
    if (lane < 32) smax[wm][(wn * NTW + n) * 32 + lane] = m;
  }
  if (a.row_max) {
    __syncthreads();
    for (int b = t; b < NT * 32 && b < a.B; b += kLmThreads) {
      float m = smax[0][b];
      for (int w = 1; w < WM; ++w) m = smax[w][b] > m ? smax[w][b] : m;
      if (m > -INFINITY) lm_atomic_max(a.row_max + b, m);
    }
  }
}

}  // namespace arbor
