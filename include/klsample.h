/*
 * klsample.h - C ABI of the MI355X (gfx950) fused token-sampling library.
 *
 * One call samples one token for each of B rows of a [B, V] logits matrix that is
 * resident in device memory.  Per row it applies, in the reference's order:
 *   repetition penalty            serving/sampling.py:47-49
 *   presence/frequency penalties  (no reference counterpart; applied after the above)
 *   greedy argmax when T == 0     serving/sampling.py:50-51
 *   temperature, top-k, top-p     serving/sampling.py:53-59
 *   the draw                      serving/sampling.py:60 (inverse CDF on a caller uniform)
 *   log-softmax + top-N logprobs  serving/sampling.py:61-63
 *
 * Conventions: the caller owns every buffer (device pointers unless stated); the
 * library never allocates, never synchronises the stream and never throws across
 * this boundary.  Every argument is validated on the host before the first HIP
 * call, so an invalid call returns a status without touching the device.
 * Functions return KLSAMPLE_OK (0) or a negative status; klsample_last_error()
 * then describes the failure (thread-local string).
 */
#ifndef KLSAMPLE_H
#define KLSAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KLSAMPLE_ABI_VERSION 3

/* status codes */
#define KLSAMPLE_OK 0
#define KLSAMPLE_ERR_INVALID_ARGUMENT (-1)
#define KLSAMPLE_ERR_UNSUPPORTED_DTYPE (-2)
#define KLSAMPLE_ERR_WORKSPACE (-3)
#define KLSAMPLE_ERR_HIP (-4)

/* logits element types */
#define KLSAMPLE_FLOAT32 0
#define KLSAMPLE_BFLOAT16 1

/* klsample_row_params.flags: the reference's double-precision tests, evaluated by the
 * caller on the original Python floats (an fp32 value alone cannot tell 0.99999999 < 1). */
#define KLSAMPLE_ROW_GREEDY 1u            /* temperature == 0       serving/sampling.py:50 */
#define KLSAMPLE_ROW_REPETITION 2u        /* repetition_penalty != 1 serving/sampling.py:47 */
#define KLSAMPLE_ROW_PRESENCE_FREQUENCY 4u /* presence or frequency penalty != 0 */
#define KLSAMPLE_ROW_TOP_P 8u             /* top_p < 1               serving/sampling.py:56 */

/* klsample_batch.options */
#define KLSAMPLE_OPT_FORCE_DENSE 1u       /* resolve every row on the multi-pass path (testing) */
#define KLSAMPLE_OPT_HISTORY_PAIRS 2u     /* history_offsets holds [begin, end) per row (2 * batch
                                             entries) into a shared id arena, instead of CSR */
#define KLSAMPLE_OPT_HOST_PARAMS 4u       /* params and history_offsets are HOST memory, read before
                                             the call returns and carried in the kernel arguments
                                             (no upload): batch <= KLSAMPLE_HOST_PARAMS_MAX_BATCH */
#define KLSAMPLE_HOST_PARAMS_MAX_BATCH 8

/* Per-row sampling parameters (32 bytes).  Mirrors SamplingParams
 * (serving/sampling.py:8-15) plus presence/frequency and the row's uniform.
 * Floats are the fp32 roundings of the Python values, which is what the reference's
 * tensor-by-scalar operations use. */
typedef struct klsample_row_params {
    float temperature;
    int32_t top_k;              /* 0 disables top-k; >= vocab keeps everything */
    float top_p;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    float uniform;              /* U[0,1) driving the inverse-CDF draw (sampled rows) */
    uint32_t flags;             /* KLSAMPLE_ROW_* */
} klsample_row_params;

/* Optional per-row diagnostics (32 bytes).  The kept set is
 * { i : s_i > cut_score } U { i : s_i == cut_score and i <= cut_index } and its
 * probabilities are exp(s_i - max_score - log_norm). */
typedef struct klsample_row_info {
    float max_score;
    float cut_score;
    int32_t cut_index;
    int32_t kept;
    double log_norm;
    int32_t path;               /* 0: resolved from chunk candidates, 1: multi-pass row path,
                                   2: top-p resolved from the chunks' histograms and scores */
    int32_t mode;               /* 0 greedy, 1 top-k, 2 top-p only, 3 full distribution */
} klsample_row_info;

/* One batched sampling call. */
typedef struct klsample_batch {
    const void *logits;         /* [batch, row_stride] of dtype; rows read, never written */
    int64_t row_stride;         /* elements between consecutive rows (>= vocab) */
    int32_t dtype;              /* KLSAMPLE_FLOAT32 | KLSAMPLE_BFLOAT16 */
    int32_t batch;              /* B >= 1 */
    int32_t vocab;              /* V >= 1 */
    int32_t num_logprobs;       /* N in [0, 256]: top-N logprobs per row */
    int32_t max_top_k;          /* max over rows of top_k (0 if none); sizes candidate slots */
    uint32_t options;           /* KLSAMPLE_OPT_* */
    const klsample_row_params *params;      /* [batch] */
    const int32_t *history_ids;             /* CSR token history; ids in [0, vocab) */
    const int32_t *history_offsets;         /* [batch + 1] (CSR), or [2 * batch] begin/end pairs with
                                               KLSAMPLE_OPT_HISTORY_PAIRS; NULL means no history */
    int64_t *token_ids;                     /* [batch] out */
    float *logprobs;                        /* [batch] out: log-softmax of the sampled token */
    int32_t *top_ids;                       /* [batch * num_logprobs] out, or NULL if N == 0 */
    float *top_logprobs;                    /* [batch * num_logprobs] out, or NULL if N == 0 */
    float *probs;                           /* optional [batch * vocab] out: final probabilities */
    klsample_row_info *row_info;            /* optional [batch] out */
    void *workspace;                        /* device scratch, see klsample_workspace_size */
    size_t workspace_bytes;
    uint32_t *history_errors;               /* optional [batch] out: history ids of penalised rows
                                               outside [0, vocab), which the call ignored (the
                                               reference's scores[ids] raises on them,
                                               serving/sampling.py:48-49); 0 for other rows */
    int32_t *history_append;                /* optional, with KLSAMPLE_OPT_HISTORY_PAIRS: row b's
                                               token is also stored at history_append[end_b] (the
                                               arena as writable memory, room reserved by the
                                               caller), so the next call's range is [begin_b,
                                               end_b + 1): the engine's prompt + generated
                                               (serving/engine.py:94) without re-uploading it */
} klsample_batch;

/* ABI version of the loaded library (KLSAMPLE_ABI_VERSION). */
int klsample_abi_version(void);

/* Bytes of device workspace a call with these sizes needs.  Writes *bytes and
 * returns KLSAMPLE_OK, or a negative status for invalid sizes.
 * No reference counterpart: the reference allocates inside torch ops per call.
 * The size grows with batch * vocab: per row a score buffer of vocab + 1 floats
 * (rounded up to 4) and 8 KB per chunk of 8,192 entries for top-p histograms, next to
 * the chunk summaries and candidate slots (the headline B = 256, V = 151,936 needs
 * ~200 MB; B = 1,024 ~800 MB).  Callers bounding their workspace split the batch. */
int klsample_workspace_size(int32_t batch, int32_t vocab, int32_t dtype, int32_t max_top_k,
                            int32_t num_logprobs, size_t *bytes);

/* Zero-fill a workspace (enqueued on `stream`, a hipStream_t).  klsample_run does not
 * require it (a call writes every workspace byte it later reads); it makes the
 * workspace contents reproducible for inspection. */
int klsample_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/* Sample one token per row; enqueued on `stream` (a hipStream_t, NULL = default).
 * Replaces Sampler.sample (serving/sampling.py:43-63), batched over rows: for row b
 * it computes what Sampler(params_b).sample(logits[b], history_b) returns, with the
 * multinomial draw of serving/sampling.py:60 replaced by the inverse CDF on
 * params[b].uniform: the smallest index i whose cumulative probability (vocab order)
 * exceeds uniform * total. */
int klsample_run(const klsample_batch *batch, void *stream);

/* Bytes of the static device scratch klsample_run_noalloc works in (per GPU). */
#define KLSAMPLE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* klsample_run without a caller workspace and without any allocation: no reference
 * counterpart; for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * results and status codes as klsample_run, except that batch->workspace must be NULL
 * and batch->workspace_bytes 0: the call works in a static device array of
 * KLSAMPLE_NOALLOC_SCRATCH_BYTES per GPU, held from the library's first use on that
 * GPU until the process ends.  A call whose klsample_workspace_size exceeds that
 * returns KLSAMPLE_ERR_WORKSPACE before touching the device.  Every call on one GPU
 * shares that GPU's array, so calls that overlap on one GPU (other streams or host
 * threads) race: issue them on one stream.  Calls no hipMalloc/hipFree. */
int klsample_run_noalloc(const klsample_batch *batch, void *stream);

/* Diagnostic timing; no reference counterpart.  With count in [1, 4], every later
 * klsample_run issued from this thread records events[i] (hipEvent_t handles owned by
 * the caller, NULL entries skipped) on its stream: events[0] before the streaming pass
 * over the logits, events[1] after it, events[2] after the per-row combine and
 * events[3] after the optional probability write-out.  The handles are copied; count
 * 0 turns recording off.  Each recording costs a stream marker, so timed calls are
 * slightly slower than unrecorded ones. */
int klsample_set_phase_events(void *const *events, int32_t count);

/* LM head fused with the sampling call (prototype).  Replaces the executor's
 * `self.model.lm_head(hidden)[:,0].float()` (serving/qwen_executor.py:238) followed by
 * the sampler: logits[b][v] = bf16(sum_k hidden[b][k] * weight[v][k]) (fp32 sums rounded
 * to bf16, as the reference's bf16 output), computed chunk by chunk with bf16 matrix
 * cores and scanned for sampling while still on chip.  The logits are also written to
 * batch->logits, which here is an OUTPUT ([batch, vocab] fp32, row_stride == vocab,
 * dtype KLSAMPLE_FLOAT32): rows the chunk summaries cannot settle, and the optional
 * probabilities, read them from there.  Every other klsample_batch field means what it
 * means for klsample_run; the workspace is sized by klsample_lmhead_workspace_size. */
typedef struct klsample_lmhead {
    const void *hidden;         /* [batch, dim] bf16, 16-byte aligned rows */
    const void *weight;         /* [vocab, dim] bf16 (lm_head.weight), 16-byte aligned */
    int32_t dim;                /* hidden size: a positive multiple of 64 */
    int32_t reserved;           /* 0 */
} klsample_lmhead;

int klsample_lmhead_workspace_size(int32_t batch, int32_t vocab, int32_t max_top_k, int32_t num_logprobs,
                                   size_t *bytes);
int klsample_lmhead_run(const klsample_batch *batch, const klsample_lmhead *head, void *stream);

/* Description of the last failure on this thread ("" if none). */
const char *klsample_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KLSAMPLE_H */
