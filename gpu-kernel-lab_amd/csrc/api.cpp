// C ABI of the token-sampling library: argument validation, launch planning and
// error reporting.  Every check runs on the host before the first HIP call.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>

#include "internal.h"

namespace {

thread_local std::string g_last_error;
thread_local kls::PhaseEvents g_phases;   // diagnostic events of this thread's calls
thread_local bool g_phases_on = false;

int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int ok() {
    g_last_error.clear();
    return KLSAMPLE_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

constexpr int32_t kMaxVocab = 1 << 24;  // masses are summed in 2^-40 fixed point in 64 bits

int check_sizes(int32_t batch, int32_t vocab, int32_t dtype, int32_t max_top_k, int32_t num_logprobs) {
    if (batch < 1 || batch > kls::kMaxBatch)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "batch must be in [1, %d] (got %d)", kls::kMaxBatch, batch);
    if (vocab < 1 || vocab > kMaxVocab)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "vocab must be in [1, %d] (got %d)", kMaxVocab, vocab);
    if (dtype != KLSAMPLE_FLOAT32 && dtype != KLSAMPLE_BFLOAT16)
        return fail(KLSAMPLE_ERR_UNSUPPORTED_DTYPE, "unsupported logits dtype code %d", dtype);
    if (max_top_k < 0) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "max_top_k must be >= 0 (got %d)", max_top_k);
    if (num_logprobs < 0 || num_logprobs > kls::kMaxLogprobs)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "num_logprobs must be in [0, %d] (got %d)", kls::kMaxLogprobs,
                    num_logprobs);
    return KLSAMPLE_OK;
}

}  // namespace

namespace kls {

bool make_plan(int32_t batch, int32_t vocab, int32_t dtype, int32_t max_top_k, int32_t num_logprobs, Plan *p,
               int32_t elems) {
    // Elements per thread: 32, the largest built variant.  Larger chunks amortise each
    // workgroup's fixed work (history table, candidate bound) in the streaming pass and
    // leave fewer chunk summaries and candidates for the row combine, which matters most
    // for small batches.
    static const int kF32[] = {32, 16, 8, 4};
    static const int kBF16[] = {32, 16, 8};
    const int *cands = dtype == KLSAMPLE_FLOAT32 ? kF32 : kBF16;
    const int ncands = dtype == KLSAMPLE_FLOAT32 ? 4 : 3;
    int e = cands[0];
    // KLSAMPLE_ELEMS_PER_THREAD pins E (tuning); ignored unless it names a built variant
    if (const char *env = getenv("KLSAMPLE_ELEMS_PER_THREAD")) {
        const int want = atoi(env);
        for (int i = 0; i < ncands; ++i)
            if (cands[i] == want) e = want;
    }
    if (elems > 0) e = elems;
    p->elems = e;
    p->chunk = kThreads * e;
    p->chunks = (vocab + p->chunk - 1) / p->chunk;
    int64_t kmax = max_top_k < vocab ? max_top_k : vocab;
    if (kmax < kTopPCandidates) kmax = kTopPCandidates;
    if (kmax < num_logprobs) kmax = num_logprobs;
    int64_t cap = (int64_t)align_up((size_t)(2 * kmax + 128), 64);
    if (cap > p->chunk) cap = p->chunk;
    p->cand_cap = (int32_t)cap;
    const size_t B = (size_t)batch, S = (size_t)p->chunks;
    size_t off = 0;
    p->off_stats = off;   off = align_up(off + B * S * sizeof(ChunkStat), 256);
    p->off_cands = off;   off = align_up(off + B * S * (size_t)cap * sizeof(Cand), 256);
    p->off_rows = off;    off = align_up(off + B * sizeof(klsample_row_info), 256);
    // ybuf rows start 16-byte aligned; the last float of a row is a spare slot that no
    // pass reads (they read up to vocab rounded up to 4)
    p->ypitch = (int32_t)align_up((size_t)vocab + 1, 4);
    p->off_ybuf = off;    off = align_up(off + B * (size_t)p->ypitch * sizeof(float), 256);
    // histograms of top-p chunks (written only by those)
    p->off_hist = off;    off = align_up(off + B * S * (size_t)kWideBins * sizeof(unsigned long long), 256);
    p->total = off;
    return (int64_t)batch * p->chunks <= INT32_MAX;
}

}  // namespace kls

extern "C" {

int klsample_abi_version(void) { return KLSAMPLE_ABI_VERSION; }

const char *klsample_last_error(void) { return g_last_error.c_str(); }

int klsample_set_phase_events(void *const *events, int32_t count) {
    if (count < 0 || count > 4) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "count must be in [0, 4] (got %d)", count);
    if (count > 0 && events == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "events must not be NULL");
    for (int i = 0; i < 4; ++i) g_phases.ev[i] = i < count ? static_cast<hipEvent_t>(events[i]) : nullptr;
    g_phases_on = count > 0;
    return ok();
}

int klsample_workspace_size(int32_t batch, int32_t vocab, int32_t dtype, int32_t max_top_k, int32_t num_logprobs,
                            size_t *bytes) {
    if (bytes == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "bytes must not be NULL");
    const int st = check_sizes(batch, vocab, dtype, max_top_k, num_logprobs);
    if (st != KLSAMPLE_OK) return st;
    kls::Plan plan;
    if (!kls::make_plan(batch, vocab, dtype, max_top_k, num_logprobs, &plan))
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "batch * chunks exceeds the grid limit");
    *bytes = plan.total;
    return ok();
}

int klsample_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
    if (workspace == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "workspace must not be NULL");
    if (workspace_bytes == 0) return ok();
    const hipError_t e = kls::launch_zero_fill(workspace, workspace_bytes, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(KLSAMPLE_ERR_HIP, "workspace init failed: %s", hipGetErrorString(e));
    return ok();
}

}  // extern "C"

namespace {

// Validates everything of a call but its workspace and fills the kernel arguments (the
// workspace pointers excepted).  Host only: no HIP call.
int prepare(const klsample_batch *b, kls::Plan *plan, kls::Args *args, int32_t elems = 0) {
    if (b == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "batch must not be NULL");
    int st = check_sizes(b->batch, b->vocab, b->dtype, b->max_top_k, b->num_logprobs);
    if (st != KLSAMPLE_OK) return st;
    if (b->logits == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "logits must not be NULL");
    if (b->row_stride < b->vocab)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "row_stride (%lld) must be >= vocab (%d)",
                    (long long)b->row_stride, b->vocab);
    if (b->params == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "params must not be NULL");
    if (b->token_ids == nullptr || b->logprobs == nullptr)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "token_ids and logprobs must not be NULL");
    if (b->num_logprobs > 0 && (b->top_ids == nullptr || b->top_logprobs == nullptr))
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "top_ids and top_logprobs are required when num_logprobs > 0");
    if (b->history_offsets != nullptr && b->history_ids == nullptr)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "history_ids must not be NULL when history_offsets is given");
    if ((b->options & ~(uint32_t)(KLSAMPLE_OPT_FORCE_DENSE | KLSAMPLE_OPT_HISTORY_PAIRS | KLSAMPLE_OPT_HOST_PARAMS)) != 0)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "unknown option bits 0x%x", b->options);
    const bool host_params = (b->options & KLSAMPLE_OPT_HOST_PARAMS) != 0;
    if (host_params && b->batch > KLSAMPLE_HOST_PARAMS_MAX_BATCH)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "KLSAMPLE_OPT_HOST_PARAMS takes at most %d rows (batch %d)",
                    KLSAMPLE_HOST_PARAMS_MAX_BATCH, b->batch);
    if (b->history_append != nullptr && !(b->options & KLSAMPLE_OPT_HISTORY_PAIRS))
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "history_append needs KLSAMPLE_OPT_HISTORY_PAIRS");
    if (b->history_append != nullptr && b->history_offsets == nullptr)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "history_append needs history ranges (history_offsets)");
    if (!kls::make_plan(b->batch, b->vocab, b->dtype, b->max_top_k, b->num_logprobs, plan, elems))
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "batch * chunks exceeds the grid limit");

    const size_t esize = b->dtype == KLSAMPLE_FLOAT32 ? 4 : 2;
    kls::Args &a = *args;
    a.logits = b->logits;
    a.row_stride = b->row_stride;
    a.B = b->batch;
    a.V = b->vocab;
    a.N = b->num_logprobs;
    a.options = b->options;
    a.params = b->params;
    a.hist_ids = b->history_ids;
    a.hist_off = b->history_offsets;
    a.inline_flags = 0;
    if (host_params) {
        // host memory: copied into the kernel arguments now, never dereferenced on the GPU
        memcpy(a.inl_params, b->params, sizeof(klsample_row_params) * (size_t)b->batch);
        a.params = nullptr;
        a.inline_flags |= kls::kInlineParams;
        if (b->history_offsets != nullptr) {
            const int n = (b->options & KLSAMPLE_OPT_HISTORY_PAIRS) ? 2 * b->batch : b->batch + 1;
            memcpy(a.inl_off, b->history_offsets, sizeof(int32_t) * (size_t)n);
            a.hist_off = nullptr;
            a.inline_flags |= kls::kInlineOffsets;
        }
    }
    a.hist_errors = b->history_errors;
    a.hist_append = b->history_append;
    a.token = b->token_ids;
    a.logprob = b->logprobs;
    a.top_ids = b->top_ids;
    a.top_lp = b->top_logprobs;
    a.probs = b->probs;
    a.row_info = b->row_info;
    a.ypitch = plan->ypitch;
    a.E = plan->elems;
    a.C = plan->chunk;
    a.S = plan->chunks;
    a.cand_cap = plan->cand_cap;
    a.vec_ok = (((uintptr_t)b->logits & 15u) == 0 && ((size_t)b->row_stride * esize) % 16 == 0) ? 1 : 0;
    a.xcd_map = (b->batch % 8 == 0) ? 1 : 0;
    a.wide_split = ((int64_t)b->batch * plan->chunks <= kls::kWideSplitGroups) ? 1 : 0;
    return KLSAMPLE_OK;
}

// Points the kernel arguments at a workspace laid out by `plan` and launches.
int launch(const klsample_batch *b, const kls::Plan &plan, kls::Args &a, void *workspace, void *stream) {
    unsigned char *ws = static_cast<unsigned char *>(workspace);
    a.stats = reinterpret_cast<kls::ChunkStat *>(ws + plan.off_stats);
    a.cands = reinterpret_cast<kls::Cand *>(ws + plan.off_cands);
    a.rows = reinterpret_cast<klsample_row_info *>(ws + plan.off_rows);
    a.ybuf = reinterpret_cast<float *>(ws + plan.off_ybuf);
    a.hist = reinterpret_cast<unsigned long long *>(ws + plan.off_hist);
    const hipError_t e = kls::launch_sample(a, b->dtype, static_cast<hipStream_t>(stream),
                                           g_phases_on ? &g_phases : nullptr);
    if (e != hipSuccess) return fail(KLSAMPLE_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
    return ok();
}

}  // namespace

extern "C" {

int klsample_run(const klsample_batch *b, void *stream) {
    kls::Plan plan;
    kls::Args a;
    const int st = prepare(b, &plan, &a);
    if (st != KLSAMPLE_OK) return st;
    if (b->workspace == nullptr) return fail(KLSAMPLE_ERR_WORKSPACE, "workspace must not be NULL");
    if (((uintptr_t)b->workspace & 255u) != 0) return fail(KLSAMPLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    if (b->workspace_bytes < plan.total)
        return fail(KLSAMPLE_ERR_WORKSPACE, "workspace too small: %zu bytes given, %zu needed", b->workspace_bytes,
                    plan.total);
    return launch(b, plan, a, b->workspace, stream);
}

int klsample_lmhead_workspace_size(int32_t batch, int32_t vocab, int32_t max_top_k, int32_t num_logprobs,
                                   size_t *bytes) {
    if (bytes == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "bytes must not be NULL");
    const int st = check_sizes(batch, vocab, KLSAMPLE_FLOAT32, max_top_k, num_logprobs);
    if (st != KLSAMPLE_OK) return st;
    kls::Plan plan;
    if (!kls::make_plan(batch, vocab, KLSAMPLE_FLOAT32, max_top_k, num_logprobs, &plan, kls::kHeadElems))
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "batch * chunks exceeds the grid limit");
    *bytes = plan.total;
    return ok();
}

int klsample_lmhead_run(const klsample_batch *b, const klsample_lmhead *h, void *stream) {
    if (h == nullptr) return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "head must not be NULL");
    if (h->hidden == nullptr || h->weight == nullptr)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "hidden and weight must not be NULL");
    if (h->dim < 64 || h->dim % 64 != 0)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "dim (%d) must be a positive multiple of 64", h->dim);
    if ((((uintptr_t)h->hidden | (uintptr_t)h->weight) & 15u) != 0)
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "hidden and weight must be 16-byte aligned");
    if (b != nullptr && (b->dtype != KLSAMPLE_FLOAT32 || b->row_stride != b->vocab))
        return fail(KLSAMPLE_ERR_INVALID_ARGUMENT, "the LM-head path writes fp32 logits with row_stride == vocab");
    kls::Plan plan;
    kls::Args a;
    const int st = prepare(b, &plan, &a, kls::kHeadElems);
    if (st != KLSAMPLE_OK) return st;
    if (b->workspace == nullptr) return fail(KLSAMPLE_ERR_WORKSPACE, "workspace must not be NULL");
    if (((uintptr_t)b->workspace & 255u) != 0) return fail(KLSAMPLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    if (b->workspace_bytes < plan.total)
        return fail(KLSAMPLE_ERR_WORKSPACE, "workspace too small: %zu bytes given, %zu needed", b->workspace_bytes,
                    plan.total);
    a.wide_split = 0;   // one workgroup per (chunk, row block) writes the histograms too
    unsigned char *ws = static_cast<unsigned char *>(b->workspace);
    a.stats = reinterpret_cast<kls::ChunkStat *>(ws + plan.off_stats);
    a.cands = reinterpret_cast<kls::Cand *>(ws + plan.off_cands);
    a.rows = reinterpret_cast<klsample_row_info *>(ws + plan.off_rows);
    a.ybuf = reinterpret_cast<float *>(ws + plan.off_ybuf);
    a.hist = reinterpret_cast<unsigned long long *>(ws + plan.off_hist);
    kls::HeadArgs head;
    head.hidden = static_cast<const uint16_t *>(h->hidden);
    head.weight = static_cast<const uint16_t *>(h->weight);
    head.logits_out = static_cast<float *>(const_cast<void *>(b->logits));
    head.dim = h->dim;
    const hipError_t e = kls::launch_lmhead(a, head, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(KLSAMPLE_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
    return ok();
}

int klsample_run_noalloc(const klsample_batch *b, void *stream) {
    kls::Plan plan;
    kls::Args a;
    const int st = prepare(b, &plan, &a);
    if (st != KLSAMPLE_OK) return st;
    if (b->workspace != nullptr || b->workspace_bytes != 0)
        return fail(KLSAMPLE_ERR_WORKSPACE, "klsample_run_noalloc takes no workspace (workspace must be NULL and "
                    "workspace_bytes 0)");
    if (plan.total > kls::kScratchBytes)
        return fail(KLSAMPLE_ERR_WORKSPACE, "this call needs %zu bytes of workspace; the static scratch holds %zu "
                    "(use klsample_run with a caller workspace)", plan.total, kls::kScratchBytes);
    void *ws = nullptr;
    const hipError_t e = kls::scratch_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return fail(KLSAMPLE_ERR_HIP, "scratch address lookup failed: %s", hipGetErrorString(e));
    return launch(b, plan, a, ws, stream);
}

}  // extern "C"
