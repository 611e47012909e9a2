/*
 * arbor_sampling.h -- C ABI of libarbor_hip.so, the MI355X (gfx950) token-sampling
 * library for ArborNet.
 *
 * One call samples one token id per row of a [batch, vocab] logits matrix:
 *
 *   logits -> temperature -> repetition / frequency / presence penalty
 *          -> optional packed allow-mask -> softmax -> top-k -> top-p -> min-p
 *          -> inverse-CDF draw against a caller-supplied uniform per row.
 *
 * Every pointer argument except `params` and the out-param of the helper calls is a
 * DEVICE pointer. The caller owns all memory, as with the reference's CUDA DLL, whose
 * kernels never allocate (ArborNet.Core/Backends/CudaBackend.cs:43-46 allocates,
 * :437-449 frees). Calls are asynchronous and stream-ordered; stream NULL is the
 * default stream. Nothing of one call outlives it: no per-call state is kept between
 * calls. The library does cache facts about each device it has seen (compute-unit count,
 * kernels' LDS limits and occupancy), filled on first use behind a mutex or atomics, so
 * concurrent calls from several host threads are safe.
 *
 * Status convention: 0 = success, negative = argument error (ARBOR_ERR_*, checked on the
 * host before anything is launched), positive = HIP runtime error code. The message of
 * the last failure on the calling thread is returned by arbor_last_error(); the managed
 * side turns a nonzero status into InvalidOperationException the way
 * ArborNet.Core/Native/PInvoke/CUDA.cs:360-364 (Check) does for CudaError.
 *
 * Per-row outcomes that only the device can see are reported through the id itself
 * (ARBOR_ID_*): all tokens masked or -inf, a NaN / +inf tempered logit, or a history id
 * >= vocab. Negative history ids are padding and are skipped, so ragged histories are
 * passed as a [batch, hist_len] matrix padded with -1.
 */
#ifndef ARBOR_SAMPLING_H
#define ARBOR_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARBOR_ABI_VERSION 1

/* dtype of the logits matrix */
#define ARBOR_DTYPE_F32 0
#define ARBOR_DTYPE_BF16 1

/* flags */
#define ARBOR_FLAG_WRITE_PROBS 1u /* write the filtered, renormalised q[batch, vocab] */

/* limits */
#define ARBOR_VOCAB_MAX 1048575     /* 2^20 - 1: ids fit the 20-bit history-table key */
#define ARBOR_HISTORY_MAX 4096      /* history entries per row */

/* status codes */
#define ARBOR_OK 0
#define ARBOR_ERR_NULL (-1)          /* a required pointer is NULL */
#define ARBOR_ERR_STRUCT_SIZE (-2)   /* params->struct_size != sizeof(arbor_sampling_params) */
#define ARBOR_ERR_SHAPE (-3)         /* batch <= 0, vocab <= 0 or > ARBOR_VOCAB_MAX, ld_logits < vocab */
#define ARBOR_ERR_DTYPE (-4)         /* dtype not ARBOR_DTYPE_* */
#define ARBOR_ERR_TEMPERATURE (-5)   /* temperature not finite and > 0 */
#define ARBOR_ERR_PENALTY (-6)       /* repetition penalty not finite and > 0; freq/presence not finite */
#define ARBOR_ERR_TOP_K (-7)         /* top_k < 0 */
#define ARBOR_ERR_TOP_P (-8)         /* top_p not in (0, 1] */
#define ARBOR_ERR_MIN_P (-9)         /* min_p not in [0, 1) */
#define ARBOR_ERR_HISTORY (-10)      /* hist_len < 0 or > ARBOR_HISTORY_MAX, or history NULL with hist_len > 0 */
#define ARBOR_ERR_MASK (-11)         /* allow_mask given with mask_words < ceil(vocab / 32) */
#define ARBOR_ERR_WORKSPACE (-12)    /* workspace NULL or smaller than arbor_sample_workspace_bytes() */
#define ARBOR_ERR_FLAGS (-13)        /* unknown flag bits, or WRITE_PROBS without out_probs */
#define ARBOR_ERR_NO_DEVICE (-14)    /* no HIP device is visible */

/* per-row sentinel ids written to out_ids */
#define ARBOR_ID_EMPTY (-1)          /* no finite tempered logit survives (all masked or -inf) */
#define ARBOR_ID_INVALID (-2)        /* a tempered, penalised, unmasked logit is NaN or +inf */
#define ARBOR_ID_BAD_HISTORY (-3)    /* the row's history holds an id >= vocab */
#define ARBOR_ID_STALLED (-4)        /* a wait between the workgroups that share the row gave up
                                        after seconds (never expected: report it as a bug) */

/*
 * Sampling parameters. A host POD passed by pointer; struct_size must equal
 * sizeof(arbor_sampling_params) so that later ABI versions can grow it.
 * A filter is disabled by top_k == 0, top_p == 1 or min_p == 0.
 */
typedef struct arbor_sampling_params {
  uint32_t struct_size;
  int32_t batch;               /* rows */
  int32_t vocab;               /* columns sampled per row */
  int32_t ld_logits;           /* elements between row starts, >= vocab and < 2^31 */
  int32_t dtype;               /* ARBOR_DTYPE_F32 or ARBOR_DTYPE_BF16 */
  float temperature;           /* z = x * (1/temperature) in fp32 */
  float repetition_penalty;    /* z > 0 ? z * (1/rp) : z * rp, once per distinct history id */
  float frequency_penalty;     /* z -= count * fp + presence_penalty, per distinct history id */
  float presence_penalty;
  int32_t top_k;
  float top_p;
  float min_p;
  int32_t hist_len;            /* history entries per row (row stride of `history`) */
  int32_t mask_words;          /* uint32 words per row of `allow_mask` (row stride) */
  uint32_t flags;              /* ARBOR_FLAG_* */
} arbor_sampling_params;

/*
 * Sample one id per row.
 *   logits      [batch, ld_logits] fp32 or bf16 (device)
 *   history     [batch, hist_len] int32 (device; may be NULL when hist_len == 0)
 *   allow_mask  [batch, mask_words] uint32, bit (t & 31) of word t >> 5 set = allowed
 *               (device; NULL = everything allowed)
 *   uniforms    [batch] fp32 in [0, 1) (device)
 *   out_ids     [batch] int32 (device)
 *   out_probs   [batch, vocab] fp32 (device; required iff flags has WRITE_PROBS)
 *   workspace   device scratch of at least arbor_sample_workspace_bytes(params) bytes;
 *               its contents need no initialisation. Calls that share a workspace must
 *               be ordered (the same stream, or synchronised).
 *   stream      hipStream_t, or NULL for the default stream
 * Replaces, for this path, the CUDA DLL entry points the managed side binds through
 * ArborNet.Core/Native/PInvoke/CUDA.cs:90-202 (NativeSoftmax :192, NativeArgMax :172,
 * NativeCumSum :178), which the reference composes into no sampler at all.
 */
int arbor_sample(const arbor_sampling_params* params, const void* logits,
                 const int32_t* history, const uint32_t* allow_mask,
                 const float* uniforms, int32_t* out_ids, float* out_probs,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * One generation step: arbor_sample, then each row's sampled id is appended to the row's
 * device history ring, so that the next step's penalties count it.
 *   logits      the last position of the model's [batch, seq, vocab] output: pass a
 *               pointer to position seq - 1 of row 0 and ld_logits = seq * vocab, which
 *               must stay below 2^31 (seq < 16744 at vocab 128256; copy the last position
 *               to a [batch, vocab] buffer for longer sequences), or the
 *               [batch, ld_logits] logits of a model that emits one position
 *   history     [batch, hist_len] int32 ring (device; -1 = empty slot); hist_len > 0
 *   positions   [batch] int32 (device): ids appended to each row so far; the sampled id
 *               goes to slot positions[b] mod hist_len and positions[b] advances. Rows
 *               whose result is a sentinel (ARBOR_ID_*) append nothing.
 *   the other arguments as for arbor_sample.
 * Streamed rows (top-k <= 64, or min-p alone) are appended by the kernel that draws them,
 * so such a step is one launch; the other paths append in a second, one-thread-per-row
 * launch.
 * No counterpart in the reference: its models return [batch, seq, vocab] logits
 * (ArborNet.Models/GPT.cs:96-111, Llama3.cs:67-74) and nothing consumes them; this is the
 * step a generation loop around those Forward calls would make.
 */
int arbor_sample_append(const arbor_sampling_params* params, const void* logits,
                        int32_t* history, int32_t* positions, const uint32_t* allow_mask,
                        const float* uniforms, int32_t* out_ids, float* out_probs,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * arbor_sample without a workspace argument and without any allocation: the library's
 * static device scratch (ARBOR_NOALLOC_SCRATCH_BYTES per device, held from the first call
 * on a device until the process ends) serves as the workspace. Arguments and results are
 * those of arbor_sample. Params whose arbor_sample_workspace_bytes() exceeds the scratch
 * return ARBOR_ERR_WORKSPACE (every path but top-k > 64 fits at vocabularies of up to
 * 262,144 ids, and at larger ones for batches of up to 256 rows; top-k > 64 fits for small
 * batches only). Every call on one device shares
 * that device's scratch: calls that overlap on one device race and must be ordered (one
 * stream, or synchronised), like calls that share a workspace.
 * No counterpart in the reference: this entry point is for callers that cannot allocate
 * device memory, such as code under HIP graph capture, tight serving loops and harnesses
 * that forbid hipMalloc.
 */
#define ARBOR_NOALLOC_SCRATCH_BYTES (16u << 20)
int arbor_sample_noalloc(const arbor_sampling_params* params, const void* logits,
                         const int32_t* history, const uint32_t* allow_mask,
                         const float* uniforms, int32_t* out_ids, float* out_probs, void* stream);

/*
 * Text of sampled ids: a tokenizer vocabulary held on the device as an id -> bytes table
 * (token_offsets [vocab + 1] int32, ascending; token_bytes the UTF-8 bytes of every token,
 * token t being bytes [token_offsets[t], token_offsets[t + 1])). Ids outside [0, vocab)
 * decode as token unk_id (nothing if unk_id is outside it too).
 *   ids           [count] int32 (device), e.g. the out_ids of arbor_sample
 *   out_offsets   [count + 1] int32 (device): where each id's text starts in out_bytes;
 *                 out_offsets[count] = total bytes (must stay below 2^31)
 *   out_bytes     device buffer of out_capacity bytes; bytes past the capacity are not
 *                 written (out_offsets[count] still reports what the text needs)
 * Replaces the per-token vocabulary scan of the reference's Decode
 * (ArborNet.Data/Tokenizers.cs:191-200 BPE, :304-313 SentencePiece: FirstOrDefault over the
 * vocabulary for each id, the unknown token when none matches): one launch for a batch.
 */
int arbor_decode(const int32_t* ids, int32_t count, const int32_t* token_offsets, const uint8_t* token_bytes,
                 int32_t vocab, int32_t unk_id, int32_t* out_offsets, uint8_t* out_bytes, size_t out_capacity,
                 void* stream);

/*
 * The embedding rows of ids, for the next forward pass of a generation loop:
 * out_rows[i, :] = table[ids[i], :], a zero row for ids outside [0, vocab) (sentinels).
 *   table     [vocab, width] fp32 or bf16 (dtype, device); out_rows [count, width], same dtype
 * Replaces ArborNet.Layers/Embedding.cs:53-57, whose Forward returns the whole weight table
 * instead of gathering the rows of its indices.
 */
int arbor_embed(const int32_t* ids, int32_t count, const void* table, int32_t vocab, int32_t width, int32_t dtype,
                void* out_rows, void* stream);

/*
 * The LM head, the step before the sampler: logits = (x · W + bias) · scale, the product
 * the reference computes as input.MatMul(weight).Add(bias) (ArborNet.Layers/Linear.cs:29,
 * on kernel.cu:56-64 matmul_kernel or hipBLAS sgemm, ArborNet.Core/Native/PInvoke/
 * ROCm.cs:224-229), on the matrix cores: operands rounded to bf16 (round to nearest even),
 * products accumulated in fp32, then + bias and × scale in fp32 (scale = 1 keeps the
 * sampler's temperature separate; scale = 1/T with the sampler at temperature 1 folds it
 * in), stored as fp32 or bf16.
 *
 * The weight is packed once (at load time) into the order the matrix instructions read:
 *   arbor_lm_head_packed_bytes  bytes of the packed weight (0 if hidden is not a positive
 *                               multiple of 128 or vocab is not in (0, ARBOR_VOCAB_MAX])
 *   arbor_lm_head_pack          weight [hidden, vocab] (ARBOR_LM_WEIGHT_HV, the reference's
 *                               Linear.weight layout, in x out, Linear.cs:14-18) or
 *                               [vocab, hidden] (ARBOR_LM_WEIGHT_VH) row-major, fp32 or bf16
 *                               -> packed (device, arbor_lm_head_packed_bytes bytes)
 *   arbor_lm_head               x [batch, ld_x] (fp32 or bf16; 16-byte aligned rows) ->
 *                               logits [batch, ld_logits] (fp32 or bf16); bias [vocab] fp32
 *                               or NULL; row_max [batch] fp32 or NULL: each row's largest
 *                               stored logit (NaN ignored). Any batch; the weight is read
 *                               once per 256 rows.
 * These allocate nothing; they run on `stream` and return once launched.
 */
#define ARBOR_LM_WEIGHT_HV 0 /* [hidden, vocab]: the reference's Linear.weight */
#define ARBOR_LM_WEIGHT_VH 1 /* [vocab, hidden] */
size_t arbor_lm_head_packed_bytes(int32_t hidden, int32_t vocab);
int arbor_lm_head_pack(const void* weight, int32_t weight_dtype, int32_t layout, int32_t hidden,
                       int32_t vocab, void* packed, void* stream);
int arbor_lm_head(const void* x, int32_t x_dtype, int32_t batch, int32_t ld_x, const void* packed,
                  const float* bias, int32_t hidden, int32_t vocab, float scale, void* logits,
                  int32_t logits_dtype, int32_t ld_logits, float* row_max, void* stream);

/* Bytes of workspace arbor_sample needs for these params (0 if params are invalid).
 * No reference counterpart: the reference's kernels need no scratch (CudaBackend.cs:43-46). */
size_t arbor_sample_workspace_bytes(const arbor_sampling_params* params);

/* Fill params with defaults for [batch, vocab] fp32 logits: temperature 1, no penalty,
 * no filter. No reference counterpart (the reference passes arguments positionally). */
void arbor_sampling_params_init(arbor_sampling_params* params, int32_t batch, int32_t vocab);

/* Number of visible HIP devices. Replaces hipGetDeviceCount as bound by
 * ArborNet.Core/Native/PInvoke/ROCm.cs:75-76 and CUDA.cs:80-81 (IsAvailable, CUDA.cs:18-30). */
int arbor_device_count(int* count);

/* Device allocation / release / copy / sync. Replace cudaMalloc, cudaFree, cudaMemcpy and
 * cudaDeviceSynchronize as bound by ArborNet.Core/Native/PInvoke/CUDA.cs:62-78 (hipMemcpy at
 * ROCm.cs:86-87). kind follows cudaMemcpyKind / hipMemcpyKind (0..4, CUDA.cs:47-54). */
int arbor_malloc(void** ptr, size_t bytes);
int arbor_free(void* ptr);
int arbor_memcpy(void* dst, const void* src, size_t bytes, int kind);
int arbor_memset(void* ptr, int value, size_t bytes);
int arbor_synchronize(void);

/* Message of the last failed call on this thread ("" if none). Replaces the message text
 * CUDA.Check builds (CUDA.cs:360-364). */
const char* arbor_last_error(void);

/* ARBOR_ABI_VERSION of the loaded library. No reference counterpart. */
int arbor_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ARBOR_SAMPLING_H */
