/*
 * sampling_oracle.c -- CPU oracle for the token-sampling step.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py load this file's library, and only as the checker. No product code
 * path calls it.
 *
 * The reference (OzzieAI-AU/ArborNet) has no sampler: no temperature, penalty, mask,
 * top-k, top-p, min-p or multinomial code exists in it. This file restates the sampling
 * contract in the reference's CPU idiom (sequential loops over one row) from the
 * primitives it does have, with their defects corrected:
 *   - temperature is a reciprocal multiply, as CpuBackend.Divide(float) = Multiply(1f/T)
 *     (ArborNet.Core/Backends/CpuBackend.cs:265);
 *   - ranking ties go to the lowest id, as ArgMax's strict '>' keeps the first maximum
 *     (CpuBackend.cs:1044-1055; CudaBackend/kernel.cu:239-255);
 *   - softmax subtracts the row max before exp (the intent of
 *     ArborNet.Core/Activations/Softmax.cs:57-61, whose Max actually sums,
 *     CpuBackend.cs:676);
 *   - the CDF is a running sum in id order accumulated in wider precision than the
 *     input, as cumsum_kernel's double accumulator (CudaBackend/kernel.cu:275-287) and
 *     CpuBackend.CumSum (CpuBackend.cs:1080-1093);
 *   - the draw is the first index whose CDF value is strictly greater than u, the
 *     intent of KMeans++ (ArborNet.Models/KMeans.cs:146-150, where ArgMin of the
 *     `cdf > r` mask inverts it).
 *
 * Arithmetic: the tempered / penalised logits z are fp32 with one rounding per
 * operation (build with -ffp-contract=off); everything after that (exp, sums, the CDF)
 * is fp64 / long double, so the oracle is the exact-arithmetic reference to within
 * ~1e-15 and rows whose outcome hinges on less than 1e-6 of probability mass are
 * reported as boundary rows rather than guessed.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/arbor_sampling.h"

/* Planted-mistake variants for the tests that pin this oracle (tests/test_oracle_pins.py
 * builds each with -DORACLE_MUTATION=n and checks that the pins catch it). 0 = the oracle. */
#ifndef ORACLE_MUTATION
#define ORACLE_MUTATION 0
#endif
#define MUT(n) (ORACLE_MUTATION == (n))

/* id in the low word of the rank key: ~id makes equal z rank by ascending id */
#define ENC_ID(i) (MUT(3) ? (uint32_t)(i) : ~(uint32_t)(i))
#define DEC_ID(c) ((int32_t)(MUT(3) ? (uint32_t)(c) : ~(uint32_t)(c)))

/* boundary bits: BOUNDARY_CDF marks a row whose id may legitimately differ from an
 * implementation that agrees with this one to within BOUNDARY_TOL of probability mass;
 * the other two bits only report that the top-p / min-p cut had tokens within
 * BOUNDARY_TOL of its threshold (their mass widens the CDF test, see sample_row). */
#define BOUNDARY_CDF 1u
#define BOUNDARY_TOP_P 2u
#define BOUNDARY_MIN_P 4u
#define BOUNDARY_TOL 1e-6

typedef struct oracle_row_info {
  int32_t id;         /* sampled id or ARBOR_ID_* sentinel */
  int32_t n_finite;   /* tokens with finite z */
  int32_t n_topk;     /* survivors of top-k */
  int32_t n_topp;     /* survivors of top-p */
  int32_t n_kept;     /* survivors of min-p: the set the draw runs over */
  int32_t cut_id;     /* id of the last kept token in rank order */
  float cut_z;        /* its z */
  float max_z;        /* largest finite z */
  uint32_t boundary;  /* BOUNDARY_* bits */
  uint32_t reserved;
  double kept_mass;   /* sum over kept tokens of exp(z - max_z) */
  double cdf_gap;     /* min over kept j of |C_j - u| */
  double flip_mass;   /* mass of tokens whose top-p / min-p membership is ambiguous, / kept_mass */
} oracle_row_info;

static inline float bf16_to_f32(uint16_t h) {
  uint32_t b = (uint32_t)h << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static inline uint32_t f32_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* Order-preserving key: numeric order of non-NaN floats maps to unsigned order. */
static inline uint32_t order_key(float z) {
  uint32_t b = f32_bits(z);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static int cmp_i32(const void* a, const void* b) {
  int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return (x > y) - (x < y);
}

/* Descending order of the composite (key << 32 | ~id): z descending, then id ascending. */
static int cmp_u64_desc(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return (x < y) - (x > y);
}

/* Partition so that the n largest composites come first (Hoare quickselect). */
static void select_top(uint64_t* v, int64_t len, int64_t n) {
  int64_t lo = 0, hi = len - 1;
  while (lo < hi) {
    uint64_t pivot = v[lo + (hi - lo) / 2];
    int64_t i = lo, j = hi;
    while (i <= j) {
      while (v[i] > pivot) i++;
      while (v[j] < pivot) j--;
      if (i <= j) {
        uint64_t t = v[i];
        v[i] = v[j];
        v[j] = t;
        i++;
        j--;
      }
    }
    if (n - 1 <= j)
      hi = j;
    else if (n - 1 >= i)
      lo = i;
    else
      break;
  }
}

/*
 * Tempered, penalised, masked logits of one row (contract steps 1-3).
 * Returns 0, ARBOR_ID_BAD_HISTORY or ARBOR_ID_INVALID.
 */
int oracle_tempered_row(const arbor_sampling_params* p, const void* logits_row,
                        const int32_t* history_row, const uint32_t* mask_row, float* z) {
  const int V = p->vocab;
  const float inv_t = 1.0f / p->temperature;
  for (int i = 0; i < V; i++) {
    float x = p->dtype == ARBOR_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)logits_row)[i])
                                           : ((const float*)logits_row)[i];
    z[i] = (MUT(7) ? x / p->temperature : x * inv_t) + 0.0f; /* + 0: -0 becomes +0, equal values tie on id */
  }
  if (p->hist_len > 0 && history_row) {
    int32_t* h = (int32_t*)malloc(sizeof(int32_t) * (size_t)p->hist_len);
    int n = 0;
    for (int j = 0; j < p->hist_len; j++) {
      int32_t t = history_row[j];
      if (t < 0) continue; /* padding */
      if (t >= V) {
        free(h);
        return ARBOR_ID_BAD_HISTORY;
      }
      h[n++] = t;
    }
    qsort(h, (size_t)n, sizeof(int32_t), cmp_i32);
    const float rp = p->repetition_penalty;
    const float inv_rp = 1.0f / rp;
    for (int j = 0; j < n;) {
      int e = j;
      while (e < n && h[e] == h[j]) e++;
      const int32_t t = h[j];
      const float count = MUT(10) ? 1.0f : (float)(e - j);
      float v = z[t];
      v = v > 0.0f ? v * (MUT(2) ? rp : inv_rp) : v * rp;
      const float pen = count * p->frequency_penalty + p->presence_penalty;
      z[t] = (MUT(1) ? v + pen : v - pen) + 0.0f;
      j = e;
    }
    free(h);
  }
  if (mask_row) {
    for (int i = 0; i < V; i++)
      if (!((mask_row[i >> 5] >> (MUT(8) ? 31 - (i & 31) : (i & 31))) & 1u)) z[i] = -INFINITY;
  }
  for (int i = 0; i < V; i++)
    if (isnan(z[i]) || z[i] == INFINITY) return ARBOR_ID_INVALID;
  return 0;
}

/* One row of the contract (steps 4-7). Scratch sizes: z[V], ck[V], ids[V]. */
static void sample_row(const arbor_sampling_params* p, const float* z, float u, int32_t* out_id,
                       float* probs_row, oracle_row_info* info, uint64_t* ck, int32_t* kept_ids,
                       double* e) {
  const int V = p->vocab;
  oracle_row_info r;
  memset(&r, 0, sizeof r);
  r.cdf_gap = INFINITY;

  int64_t nf = 0;
  for (int i = 0; i < V; i++)
    if (z[i] != -INFINITY)
      ck[nf++] = ((uint64_t)order_key(z[i]) << 32) | ENC_ID(i);
  r.n_finite = (int32_t)nf;
  if (probs_row)
    for (int i = 0; i < V; i++) probs_row[i] = 0.0f;
  if (nf == 0) {
    r.id = ARBOR_ID_EMPTY;
    *out_id = r.id;
    if (info) *info = r;
    return;
  }

  /* top-k: the n first tokens of the ranking (z desc, id asc) */
  int64_t n = nf;
  if (p->top_k > 0 && p->top_k < nf) {
    n = p->top_k;
    select_top(ck, nf, n);
  }
  qsort(ck, (size_t)n, sizeof(uint64_t), cmp_u64_desc);
  r.n_topk = (int32_t)n;

  const double zmax = (double)z[DEC_ID(ck[0])];
  r.max_z = (float)zmax;
  long double ek = 0.0L;
  for (int64_t i = 0; i < n; i++) {
    e[i] = exp((double)z[DEC_ID(ck[i])] - zmax);
    ek += e[i];
  }

  /* top-p over the renormalised top-k survivors: shortest prefix with mass >= top_p */
  long double flip = 0.0L;
  int64_t lp = n;
  if (p->top_p < 1.0f) {
    const double tp = (double)p->top_p;
    long double cum = 0.0L;
    int64_t cut = -1;
    for (int64_t j = 0; j < n; j++) {
      cum += e[j];
      const double frac = (double)(cum / ek);
      /* token j+1 is kept iff frac_j < top_p: ambiguous when frac_j is near top_p */
      if (fabs(frac - tp) < BOUNDARY_TOL && j + 1 < n) {
        r.boundary |= BOUNDARY_TOP_P;
        flip += e[j + 1];
      }
      if (cut < 0 && (MUT(5) ? frac > tp : frac >= tp)) cut = j;
    }
    lp = cut < 0 ? n : cut + 1;
  }
  r.n_topp = (int32_t)lp;

  /* min-p over the top-p survivors: q_i >= min_p * max q, i.e. exp(z_i - zmax) >= min_p */
  int64_t lk = lp;
  if (p->min_p > 0.0f) {
    const double mp = (double)p->min_p;
    lk = 0;
    for (int64_t j = 0; j < lp; j++) {
      if (fabs(e[j] / mp - 1.0) < BOUNDARY_TOL) {
        r.boundary |= BOUNDARY_MIN_P;
        flip += e[j];
      }
      if ((MUT(9) ? e[j] / (double)ek : e[j]) >= mp) lk = j + 1;
    }
  }
  r.n_kept = (int32_t)lk;
  r.cut_id = DEC_ID(ck[lk - 1]);
  r.cut_z = z[r.cut_id];

  /* draw: CDF over the kept set in ascending id order; first C_j > u */
  long double ekept = 0.0L;
  for (int64_t j = 0; j < lk; j++) {
    kept_ids[j] = DEC_ID(ck[j]);
    ekept += e[j];
  }
  r.kept_mass = (double)ekept;
  if (!MUT(6)) qsort(kept_ids, (size_t)lk, sizeof(int32_t), cmp_i32);
  long double cum = 0.0L;
  int32_t pick = kept_ids[lk - 1]; /* no C_j > u through rounding: the last kept id */
  int found = 0;
  for (int64_t j = 0; j < lk; j++) {
    const int32_t t = kept_ids[j];
    const double et = exp((double)z[t] - zmax);
    cum += et;
    const double c = (double)(cum / ekept);
    const double gap = fabs(c - (double)u);
    if (gap < r.cdf_gap) r.cdf_gap = gap;
    if (!found && (MUT(4) ? c >= (double)u : c > (double)u)) {
      pick = t;
      found = 1;
    }
    if (probs_row) probs_row[t] = (float)(et / (double)ekept);
  }
  /* Adding or removing ambiguous tokens of total mass F moves every C_j by at most
   * F / kept_mass, and a flipped token's own CDF interval is that narrow too. */
  r.flip_mass = (double)(flip / ekept);
  if (r.cdf_gap < BOUNDARY_TOL + r.flip_mass) r.boundary |= BOUNDARY_CDF;
  r.id = pick;
  *out_id = pick;
  if (info) *info = r;
}

/*
 * Sample rows [row0, row0 + nrows) of a host-resident batch. Arguments mirror
 * arbor_sample with host pointers; out_probs and info may be NULL. nthreads > 1 splits
 * rows over OpenMP threads (rows are independent). Returns 0 or an ARBOR_ERR_* code.
 */
int oracle_sample(const arbor_sampling_params* p, const void* logits, const int32_t* history,
                  const uint32_t* mask, const float* uniforms, int32_t* out_ids,
                  float* out_probs, oracle_row_info* info, int row0, int nrows,
                  int nthreads) {
  if (!p || !logits || !uniforms || !out_ids) return ARBOR_ERR_NULL;
  if (p->vocab <= 0 || p->batch <= 0 || p->ld_logits < p->vocab) return ARBOR_ERR_SHAPE;
  if (row0 < 0 || nrows < 0 || row0 + nrows > p->batch) return ARBOR_ERR_SHAPE;
  const size_t elt = p->dtype == ARBOR_DTYPE_BF16 ? 2 : 4;
  const int V = p->vocab;
  int status = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    float* z = (float*)malloc(sizeof(float) * (size_t)V);
    uint64_t* ck = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
    int32_t* kept = (int32_t*)malloc(sizeof(int32_t) * (size_t)V);
    double* e = (double*)malloc(sizeof(double) * (size_t)V);
#pragma omp for schedule(dynamic, 1)
    for (int b = row0; b < row0 + nrows; b++) {
      const int local = b - row0;
      const void* xrow = (const char*)logits + (size_t)b * (size_t)p->ld_logits * elt;
      const int32_t* hrow = history ? history + (size_t)b * (size_t)p->hist_len : NULL;
      const uint32_t* mrow = mask ? mask + (size_t)b * (size_t)p->mask_words : NULL;
      float* prow = out_probs ? out_probs + (size_t)local * (size_t)V : NULL;
      oracle_row_info* irow = info ? info + local : NULL;
      const int st = oracle_tempered_row(p, xrow, hrow, mrow, z);
      if (st != 0) {
        out_ids[local] = st;
        if (prow)
          for (int i = 0; i < V; i++) prow[i] = 0.0f;
        if (irow) {
          memset(irow, 0, sizeof *irow);
          irow->id = st;
        }
        continue;
      }
      sample_row(p, z, uniforms[b], &out_ids[local], prow, irow, ck, kept, e);
    }
    free(z);
    free(ck);
    free(kept);
    free(e);
  }
  return status;
}

int oracle_info_size(void) { return (int)sizeof(oracle_row_info); }
