// Internal declarations shared by the C ABI (api.cpp) and the gfx950 kernels (sampling.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "klsample.h"

namespace kls {

constexpr int kThreads = 256;          // workgroup size of every kernel (4 wave64s)
constexpr int kWaves = kThreads / 64;
constexpr int kSortCap = 2048;         // candidates a row can resolve in LDS
constexpr int kTopPCandidates = 64;    // per-chunk candidates for rows with top-p but no top-k
constexpr int kMaxLogprobs = 256;      // largest supported num_logprobs
constexpr int kMaxBatch = 65536;       // rows per call
constexpr int kMaxChunksLds = 4096;    // chunks per row the candidate combine indexes in LDS

// Chunks of top-p rows also write a log-space histogram and their final scores, for
// rows whose kept set reaches past the candidates: bin j of a chunk holds the
// entries with floor(y * kWideCells) == G - j, G = floor(m_c * kWideCells) for the
// chunk max m_c (the last bin everything further down).  Each bin is one 64-bit word:
// the entry count above bit kWideCountShift, below it the sum of the entries'
// fixed-point weights exp(y - G / kWideCells) in units of 2^-kWideMassBits.
constexpr int kInlineRows = KLSAMPLE_HOST_PARAMS_MAX_BATCH;
constexpr int32_t kInlineParams = 1;
constexpr int32_t kInlineOffsets = 2;
constexpr int kWideBins = 1024;
constexpr float kWideCells = 32.f;       // bins per unit of score (natural log)
constexpr int kWideCountShift = 50;
constexpr int kWideMassBits = 36;
constexpr float kWideMaxScore = 262144.f; // |chunk max| below this keeps the grid exact in fp32
constexpr int kWideMaxChunks = 512;      // chunks per row the wide resolution indexes in LDS
constexpr int kWideSplitGroups = 512;    // at most this many (row, chunk) workgroups: the
                                         // histograms come from a second workgroup per chunk

// ChunkStat::flags
constexpr int32_t kChunkOverflow = 1;    // candidates exceeded the slot capacity
constexpr int32_t kChunkWide = 2;        // histogram and final scores written (top-p chunk)

// Row classes; every row of a batch is one of these.
enum RowMode : int { kGreedy = 0, kTopK = 1, kTopP = 2, kFull = 3 };

// Per-chunk summary written by the streaming pass (32 bytes).
struct ChunkStat {
    float m;          // chunk max of the transformed scores (greedy / top-p / full rows)
    int32_t arg;      // lowest index attaining m (greedy rows)
    float y_thr;      // every element of the chunk with score >= y_thr is a candidate
    int32_t ncand;    // candidates written (capped at the slot capacity)
    double z;         // sum of exp(s - m) over the chunk
    int32_t flags;    // kChunkOverflow | kChunkWide
    int32_t nfinite;  // elements with a finite score (greedy / top-p / full rows)
};

struct Cand {
    float y;          // final-space score (penalised, divided by T for sampled rows)
    int32_t idx;      // vocab index
};

// Launch plan: how a row is split into chunks and how the workspace is laid out.
struct Plan {
    int32_t elems;    // elements per thread (E)
    int32_t chunk;    // elements per chunk (kThreads * E)
    int32_t chunks;   // chunks per row (S)
    int32_t cand_cap; // candidate slots per chunk
    int32_t ypitch;   // floats per row of the dense path's score buffer
    size_t off_stats, off_cands, off_rows, off_ybuf, off_hist, total;
};

// elems > 0 pins the elements per thread (the LM-head path's chunks)
bool make_plan(int32_t batch, int32_t vocab, int32_t dtype, int32_t max_top_k, int32_t num_logprobs,
               Plan *plan, int32_t elems = 0);

// Everything a kernel needs, passed by value.
struct Args {
    const void *logits;
    int64_t row_stride;
    int32_t B, V, N;
    uint32_t options;
    const klsample_row_params *params;
    const int32_t *hist_ids;
    const int32_t *hist_off;
    uint32_t *hist_errors;   // optional [B]: out-of-range history ids of penalised rows
    int32_t *hist_append;    // optional: row b's token also stored at hist_append[end_b]
    int64_t *token;
    float *logprob;
    int32_t *top_ids;
    float *top_lp;
    float *probs;
    klsample_row_info *row_info;
    ChunkStat *stats;
    Cand *cands;           // per (row, chunk): cand_cap slots
    klsample_row_info *rows;
    float *ybuf;           // per row ypitch final scores (top-p chunks, dense row path)
    unsigned long long *hist;  // per (row, chunk) kWideBins histogram words of a top-p chunk
    int32_t ypitch;        // vocab + 1 rounded up to a multiple of 4 (the last float is a spare slot)
    int32_t E, C, S, cand_cap;
    int32_t vec_ok;   // 16-byte vector loads are legal for every row
    int32_t xcd_map;  // place all chunks of a row on one XCD
    int32_t wide_split;  // top-p chunks' histograms from a second workgroup each (small grids)
    // Small batches may carry their row parameters and history offsets here, in the
    // kernel arguments, instead of in device memory (kInlineParams / kInlineOffsets).
    int32_t inline_flags;
    klsample_row_params inl_params[kInlineRows];
    int32_t inl_off[2 * kInlineRows];
};

// Caller-owned hipEvent_t handles recorded around the kernels of a call (diagnostics):
// ev[0] before the streaming pass, ev[1] after it, ev[2] after the row combine,
// ev[3] after the optional probability write-out.  NULL entries are skipped.
struct PhaseEvents {
    hipEvent_t ev[4];
};

hipError_t launch_sample(const Args &args, int32_t dtype, hipStream_t stream, const PhaseEvents *phases);

// LM head fused with the streaming pass: logits[b][v] = bf16(sum_k hidden[b][k] * weight[v][k])
// computed per (vocabulary chunk of kHeadChunk, block of kHeadRows rows) with bf16 MFMA,
// materialised into `logits_out` (= Args::logits, fp32 [B][V]) and scanned from LDS.
constexpr int kHeadElems = 4;                     // chunk = kThreads * kHeadElems vocabulary rows
constexpr int kHeadRows = 16;                     // batch rows per workgroup (one MFMA column tile)
struct HeadArgs {
    const uint16_t *hidden;   // [B][dim] bf16
    const uint16_t *weight;   // [V][dim] bf16
    float *logits_out;        // [B][V] fp32
    int32_t dim;              // multiple of 64
};
hipError_t launch_lmhead(const Args &args, const HeadArgs &head, hipStream_t stream);
hipError_t launch_zero_fill(void *ptr, size_t bytes, hipStream_t stream);

// Workspace of klsample_run_noalloc: a static device array of kScratchBytes per GPU.
// scratch_workspace returns its device address on the device of `stream` (the current
// device for the NULL stream), taken once per device with hipGetSymbolAddress.
constexpr size_t kScratchBytes = KLSAMPLE_NOALLOC_SCRATCH_BYTES;
hipError_t scratch_workspace(hipStream_t stream, void **ptr);

}  // namespace kls
