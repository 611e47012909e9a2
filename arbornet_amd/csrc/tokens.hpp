// tokens.hpp -- the two steps around a sampled id in a generation loop: turning ids into
// text (a CSR id -> bytes table resident on the device) and gathering the embedding rows of
// the ids for the next forward pass. Both are byte moves bound by HBM (or by launch latency
// at a generation step's few hundred ids); nothing here is arithmetic.
#pragma once

#include "args.hpp"
#include "block_ops.hpp"

namespace arbor {

constexpr int kDecodeBlock = 1024;

// One workgroup walks the ids in rounds of 1024: each thread looks up its id's byte range,
// a block scan places the ranges one after another, and each thread copies its bytes.
// out_offsets[i] is where id i's text starts, out_offsets[count] the total; bytes past
// `capacity` are not written (the total still tells the caller how much room was needed).
__global__ void __launch_bounds__(kDecodeBlock) decode_kernel(const int32_t* ids, int count,
                                                              const int32_t* token_offsets,
                                                              const uint8_t* token_bytes, int vocab, int unk_id,
                                                              int32_t* out_offsets, uint8_t* out, size_t capacity) {
  __shared__ uint64_t scratch[kDecodeBlock / kWave];
  const int t = threadIdx.x;
  uint64_t base = 0;
  for (int c0 = 0; c0 < count; c0 += kDecodeBlock) {
    const int i = c0 + t;
    uint64_t len = 0;
    int32_t src = 0;
    if (i < count) {
      const int32_t id = ids[i];
      const int32_t tok = (id >= 0 && id < vocab) ? id : unk_id;  // outside the vocabulary: the unknown token
      if (tok >= 0 && tok < vocab) {
        src = token_offsets[tok];
        len = (uint64_t)(token_offsets[tok + 1] - src);
      }
    }
    uint64_t total;
    const uint64_t pos = base + block_scan_excl<kDecodeBlock, uint64_t>(len, scratch, &total);
    if (i < count) {
      out_offsets[i] = (int32_t)pos;
      for (uint64_t k = 0; k < len && pos + k < capacity; ++k) out[pos + k] = token_bytes[src + k];
    }
    base += total;
  }
  if (t == 0) out_offsets[count] = (int32_t)base;
}

// Row gather: out[i, :] = table[ids[i], :] (zeros for ids outside [0, vocab)). Workgroup
// (x, i) copies 16-byte units x * 256 .. of row i; UNITS: the row is made of whole,
// aligned 16-byte units, else it is copied element by element.
template <bool UNITS>
__global__ void __launch_bounds__(256) embed_kernel(const int32_t* ids, const unsigned char* table, int vocab,
                                                    int row_bytes, unsigned char* out) {
  const int i = blockIdx.y;
  const int32_t id = ids[i];
  const bool valid = id >= 0 && id < vocab;
  const unsigned char* src = table + (size_t)(valid ? id : 0) * (size_t)row_bytes;
  unsigned char* dst = out + (size_t)i * (size_t)row_bytes;
  if (UNITS) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const int u = blockIdx.x * 256 + threadIdx.x;
    if (u * 16 < row_bytes) {
      const u4 v = valid ? __builtin_nontemporal_load(reinterpret_cast<const u4*>(src) + u) : u4{0u, 0u, 0u, 0u};
      __builtin_nontemporal_store(v, reinterpret_cast<u4*>(dst) + u);
    }
  } else {
    for (int b = blockIdx.x * 256 + threadIdx.x; b < row_bytes; b += gridDim.x * 256)
      dst[b] = valid ? src[b] : (unsigned char)0;
  }
}

}  // namespace arbor
