/*
 * synth.c -- seeded synthetic sampling workloads (logits, histories, allow-masks,
 * uniforms), shared bit-for-bit by the benchmark, the tests and the smoke check.
 *
 * Determinism: every value is a function of (seed, stream, row) only, so any subset of
 * rows can be regenerated alone. Only IEEE basic operations are used (+ - * / sqrt,
 * no libm transcendental, no FMA contraction: build with -ffp-contract=off), so the
 * same bits come out on any x86-64 host regardless of libm or CPU dispatch.
 *
 * RNG: SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
 * generators", OOPSLA 2014). Normals: Box-Muller in fp64, rounded to fp32.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull
#define STREAM_MUL 0xD1B54A32D192ED03ull

enum { S_LOGITS = 1, S_SPIKES = 2, S_HISTORY = 3, S_MASK = 4, S_UNIFORM = 5, S_PERM = 6 };

typedef struct { uint64_t s; } rng_t;

static inline uint64_t next_u64(rng_t* r) {
  uint64_t z = (r->s += GOLDEN);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline rng_t rng_for(uint64_t seed, uint64_t stream, uint64_t row) {
  rng_t r;
  r.s = seed ^ (row * GOLDEN) ^ (stream * STREAM_MUL);
  next_u64(&r); /* decorrelate nearby states */
  return r;
}

/* uniform double in (0, 1]: 53 random bits */
static inline double next_open01(rng_t* r) { return ((double)(next_u64(r) >> 11) + 1.0) * 0x1.0p-53; }
/* uniform double in [0, 1) */
static inline double next_01(rng_t* r) { return (double)(next_u64(r) >> 11) * 0x1.0p-53; }
/* uniform integer in [0, n) by multiply-high */
static inline uint32_t next_below(rng_t* r, uint32_t n) {
  return (uint32_t)(((next_u64(r) >> 32) * (uint64_t)n) >> 32);
}

/* natural log for x > 0 from atanh series: log m = 2 atanh((m-1)/(m+1)), m in [sqrt(.5), sqrt(2)) */
static double det_log(double x) {
  int e;
  double m = frexp(x, &e); /* exact: x = m * 2^e, m in [0.5, 1) */
  if (m < 0.70710678118654752440) {
    m *= 2.0;
    e -= 1;
  }
  const double t = (m - 1.0) / (m + 1.0);
  const double t2 = t * t;
  double s = 1.0 / 23.0;
  for (int k = 21; k >= 1; k -= 2) s = 1.0 / (double)k + t2 * s;
  const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
  return (double)e * ln2_hi + (2.0 * t * s + (double)e * ln2_lo);
}

/* sin and cos of (pi/2) * f for f in [0, 1), Taylor to degree 21 / 20 */
static void det_sincos_quarter(double f, double* s, double* c) {
  const double a = f * 1.57079632679489661923;
  const double a2 = a * a;
  double ps = 1.0, pc = 1.0;
  for (int k = 21; k >= 3; k -= 2) ps = 1.0 - a2 / ((double)k * (double)(k - 1)) * ps;
  for (int k = 20; k >= 2; k -= 2) pc = 1.0 - a2 / ((double)k * (double)(k - 1)) * pc;
  *s = a * ps;
  *c = pc;
}

/* (cos, sin) of 2*pi*u for u in [0, 1) */
static void det_cossin_2pi(double u, double* c, double* s) {
  const double v = u * 4.0; /* exact */
  const int q = (int)v;
  const double f = v - (double)q; /* exact */
  double sf, cf;
  det_sincos_quarter(f, &sf, &cf);
  switch (q & 3) {
    case 0: *c = cf; *s = sf; break;
    case 1: *c = -sf; *s = cf; break;
    case 2: *c = -cf; *s = -sf; break;
    default: *c = sf; *s = -cf; break;
  }
}

static inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu)) return (uint16_t)((b >> 16) | 0x40);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

/*
 * Rows [row0, row0+nrows) of fp32 logits: x = sigma * N(0,1)
 *   + (n_spikes distinct ids per row) U(spike_lo, spike_hi)
 *   - zipf_s * ln(rank(id)), rank = 1 + perm[id] (perm shared by all rows of a seed).
 * out is [nrows, ld]; columns [vocab, ld) are left untouched. perm may be NULL if
 * zipf_s == 0.
 */
void synth_logits_f32(uint64_t seed, int row0, int nrows, int vocab, int ld, double sigma,
                      int n_spikes, double spike_lo, double spike_hi, double zipf_s,
                      const int32_t* perm, float* out) {
  for (int b = 0; b < nrows; b++) {
    const uint64_t row = (uint64_t)(row0 + b);
    float* x = out + (size_t)b * (size_t)ld;
    rng_t r = rng_for(seed, S_LOGITS, row);
    for (int i = 0; i < vocab; i += 2) {
      const double u1 = next_open01(&r), u2 = next_01(&r);
      const double rad = sqrt(-2.0 * det_log(u1));
      double c, s;
      det_cossin_2pi(u2, &c, &s);
      double v0 = sigma * rad * c, v1 = sigma * rad * s;
      if (zipf_s != 0.0) {
        v0 -= zipf_s * det_log((double)(perm[i] + 1));
        if (i + 1 < vocab) v1 -= zipf_s * det_log((double)(perm[i + 1] + 1));
      }
      x[i] = (float)v0;
      if (i + 1 < vocab) x[i + 1] = (float)v1;
    }
    if (n_spikes > 0) {
      rng_t rs = rng_for(seed, S_SPIKES, row);
      int32_t chosen[256];
      const int ns = n_spikes < 256 ? n_spikes : 256;
      for (int j = 0; j < ns && j < vocab; j++) {
        int32_t t;
        int dup;
        do {
          t = (int32_t)next_below(&rs, (uint32_t)vocab);
          dup = 0;
          for (int q = 0; q < j; q++) dup |= chosen[q] == t;
        } while (dup);
        chosen[j] = t;
        const double amp = spike_lo + (spike_hi - spike_lo) * next_01(&rs);
        x[t] = (float)((double)x[t] + amp);
      }
    }
  }
}

/* Same values as synth_logits_f32, rounded to bf16 (round to nearest even). */
void synth_logits_bf16(uint64_t seed, int row0, int nrows, int vocab, int ld, double sigma,
                       int n_spikes, double spike_lo, double spike_hi, double zipf_s,
                       const int32_t* perm, float* scratch_row, uint16_t* out) {
  for (int b = 0; b < nrows; b++) {
    synth_logits_f32(seed, row0 + b, 1, vocab, vocab, sigma, n_spikes, spike_lo, spike_hi, zipf_s,
                     perm, scratch_row);
    uint16_t* y = out + (size_t)b * (size_t)ld;
    for (int i = 0; i < vocab; i++) y[i] = f32_to_bf16_rne(scratch_row[i]);
  }
}

/* Seeded permutation of [0, vocab) (Fisher-Yates), used as the Zipf rank table. */
void synth_permutation(uint64_t seed, int vocab, int32_t* perm) {
  for (int i = 0; i < vocab; i++) perm[i] = i;
  rng_t r = rng_for(seed, S_PERM, 0);
  for (int i = vocab - 1; i > 0; i--) {
    const int j = (int)next_below(&r, (uint32_t)(i + 1));
    const int32_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
}

/* History [nrows, hist_len]: position p copies an earlier id of its row with
 * probability repeat_p, else draws uniformly from [0, vocab). */
void synth_history(uint64_t seed, int row0, int nrows, int hist_len, int vocab, double repeat_p,
                   int32_t* out) {
  for (int b = 0; b < nrows; b++) {
    rng_t r = rng_for(seed, S_HISTORY, (uint64_t)(row0 + b));
    int32_t* h = out + (size_t)b * (size_t)hist_len;
    for (int p = 0; p < hist_len; p++) {
      if (p > 0 && next_01(&r) < repeat_p)
        h[p] = h[next_below(&r, (uint32_t)p)];
      else
        h[p] = (int32_t)next_below(&r, (uint32_t)vocab);
    }
  }
}

/* Allow-mask [nrows, words], LSB-first: one contiguous block of block_len ids at a
 * seeded offset plus n_scatter seeded ids. */
void synth_mask(uint64_t seed, int row0, int nrows, int vocab, int words, int block_len,
                int n_scatter, uint32_t* out) {
  for (int b = 0; b < nrows; b++) {
    rng_t r = rng_for(seed, S_MASK, (uint64_t)(row0 + b));
    uint32_t* m = out + (size_t)b * (size_t)words;
    memset(m, 0, sizeof(uint32_t) * (size_t)words);
    const int span = vocab - block_len + 1;
    const int off = span > 0 ? (int)next_below(&r, (uint32_t)span) : 0;
    for (int t = off; t < off + block_len && t < vocab; t++) m[t >> 5] |= 1u << (t & 31);
    for (int j = 0; j < n_scatter; j++) {
      const int t = (int)next_below(&r, (uint32_t)vocab);
      m[t >> 5] |= 1u << (t & 31);
    }
  }
}

/* Uniforms [nrows]: 24 random bits, (k >> 40) * 2^-24 in [0, 1). */
void synth_uniforms(uint64_t seed, int row0, int nrows, float* out) {
  for (int b = 0; b < nrows; b++) {
    rng_t r = rng_for(seed, S_UNIFORM, (uint64_t)(row0 + b));
    out[b] = (float)(next_u64(&r) >> 40) * 0x1.0p-24f;
  }
}

/* Test hooks for the deterministic math (compared against libm in the tests). */
double synth_det_log(double x) { return det_log(x); }
void synth_det_cossin(double u, double* c, double* s) { det_cossin_2pi(u, c, s); }
